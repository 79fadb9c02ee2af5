// INT8 x INT8 -> INT32 GEMM with the W8A8 epilogue, for gfx950.
//
// Contract (reference: turing_utils::int8_linear, kernel/csrc/turing/w4a8.cu
// :1185-1219 with the CUTLASS EVT epilogue of :480-525):
//   acc[m][n] = sum_k a[m][k] * w[n][k]            (exact int32)
//   out[m][n] = bf16_rn(((float(acc) * as[m]) * ws[n]) + bias[n])
// The same fp32 value is also written rounded once to fp16 (RNE, NaN as
// 0x7e00) or unrounded as fp32: the output_dtype of the plugin's GEMM call
// (comfyui_turing_utils/quantization/dispatch.py:538-615).
// a and w are both K-contiguous ("TN"), so every MFMA operand is a 16-byte
// contiguous load along K.
//
// MI355X mapping
//   * Workgroup tile 256 (n) x 256 (m) x 128 (k), 8 wave64 in a 2 (n) x 4 (m)
//     grid, each wave owning a 128 x 64 output tile = 2 x 8 x 4
//     v_mfma_i32_16x16x64_i8 per K step (128 accumulator registers).  One
//     workgroup per CU, two waves per SIMD, so one wave's LDS fragment reads
//     and barrier waits overlap the other's MFMAs.
//   * The W tile is the MFMA A operand and the activation tile the B operand,
//     so each lane ends with 4 consecutive output columns of one row.  The
//     bf16 epilogue loads the tile's scales and bias in one batch, writes
//     each wave's 64 x 128 bf16 tile to LDS (the ring is free by then) and
//     stores whole 256-byte rows, 16 bytes per lane; the INT32 output stores
//     16 bytes per 16 x 16 sub-tile row directly.  Output stores are
//     non-temporal: written once and never re-read here, they would otherwise
//     evict the activation and weight panels that neighbouring tiles re-read
//     from L2 (measured: 15 % at qkv and ffn-up).
//   * K steps of 128 bytes through a 2-stage LDS ring (2 x 64 KiB) filled by
//     buffer_load_dwordx4 ... lds (direct to LDS, no staging registers) one
//     step ahead of the MFMAs.  Within a step the two 64-deep fragment sets
//     are double-buffered in registers: slice 1 is read from LDS while slice
//     0 is on the MFMAs, and slice 0 of the next step while slice 1 is.  Rows
//     are 128 B; the 16-byte chunk index is XOR-swizzled with row bits 1..3
//     (applied through each lane's source address).  A partial last K step
//     (K % 128 != 0) is staged through registers with zero fill.
//   * Tiles are renumbered so each XCD (workgroup id mod 8) owns a contiguous
//     range, walked in groups of 4 m-tiles for L2 reuse of the A and W panels
//     (measured best among 2, 4, 6, 8, 16 and 32 once the output no longer
//     pollutes L2).
#include <type_traits>

#include "tu_common.h"

namespace tu {
namespace {

// Workgroup tile: BM activation rows x BN weight rows (output columns).
// 256 x 256, or for grids that those would fill in few, partly empty rounds
// (the tile policy) 128 x 256 or 256 x 192; the wave grid stays the same.
constexpr int kBK = 128;  // bytes of K per step (two 64-deep MFMA slices)
// Waves per workgroup: 2 along the weight rows x kWavesM along the activation
// rows; each wave owns a 128 x (256 / kWavesM) output tile.
#ifndef TU_GEMM_WAVES_M
#define TU_GEMM_WAVES_M 4
#endif
constexpr int kWavesM = TU_GEMM_WAVES_M;
constexpr int kWaves = 2 * kWavesM;
constexpr int kThreads = 64 * kWaves;
constexpr int kGroupM = 4;
#ifndef TU_GEMM_HALF_TILE_COST
#define TU_GEMM_HALF_TILE_COST 0.635
#endif

// Geometry of a workgroup tile with BM activation rows and BN weight rows.
template <int BM, int BN>
struct Tile {
    static_assert((BM == 256 && (BN == 256 || BN == 192)) || (BM == 128 && BN == 256), "tile of 256 x 256, 128 x 256 or 256 x 192");
    static constexpr int kFragsM = BM / kWavesM / 16;  // 16-row activation fragments per wave
    static constexpr int kFragsN = BN / 2 / 16;        // 16-row weight fragments per wave (its half of the tile)
    static constexpr int kMma = kFragsN * kFragsM;     // MFMAs per 64-deep slice and wave
    // MFMAs of slice 0 issued before the step's barrier, covering the latency
    // of slice 1's LDS reads (the rest cover the next step's loads)
    static constexpr int kPre = kMma / 2;
    static constexpr int kABlocks = BM * 128 / 1024 / kWaves;   // 1 KiB activation blocks per wave and step
    static constexpr int kWBlocks = BN * 128 / 1024 / kWaves;   // 1 KiB weight blocks per wave and step
    static constexpr int kBlocks = kABlocks > kWBlocks ? kABlocks : kWBlocks;
    static constexpr int kLoads = kABlocks + kWBlocks;          // vector-memory loads per wave and step
    static constexpr int kStageBytes = (BM + BN) * 128;         // activation panel + weight panel
    static constexpr int kChunksA = BM * 8 / kThreads;          // 16-byte chunks per thread, register path
    static constexpr int kChunksW = BN * 8 / kThreads;
    static constexpr int kChunks = kChunksA > kChunksW ? kChunksA : kChunksW;
    static constexpr int kRows = 16 * kFragsM;                  // activation rows per wave
    // LDS: the K-step ring, and after the main loop each wave's 16-bit output
    // tile (kRows rows of 256 bytes) staged for row-wide stores
    static constexpr int kLdsBytes = 2 * kStageBytes > kWaves * kRows * 256 ? 2 * kStageBytes : kWaves * kRows * 256;
};

// LDS panel layout: 128-byte rows, the 16-byte chunk index XOR-swizzled with
// row bits 1..3 (measured bank-conflict free for 16 lanes reading one chunk
// of 16 consecutive rows; 64-byte rows with a 2-bit swizzle were not).
__device__ __forceinline__ int swz(int row, int chunk) { return row * kBK + ((chunk ^ ((row >> 1) & 7)) << 4); }

template <int BM, int BN>
struct TileLoad {
    i32x4 a[Tile<BM, BN>::kChunksA];
    i32x4 w[Tile<BM, BN>::kChunksW];
};

// Loads the BM x 128 B activation and BN x 128 B weight panels of step k0
// into registers.  Rows past the end are clamped (their results are never
// stored); columns past K are zero.
template <int BM, int BN>
__device__ __forceinline__ void load_tiles(TileLoad<BM, BN> &t, const int8_t *__restrict__ a,
                                           const int8_t *__restrict__ w, int64_t m0, int64_t n0,
                                           int64_t m, int64_t n, int64_t k, int64_t k0, int tid) {
#pragma unroll
    for (int i = 0; i < Tile<BM, BN>::kChunks; ++i) {
        const int id = tid + kThreads * i;
        const int row = id >> 3;
        const int64_t kk = k0 + (id & 7) * 16;
        if (i < Tile<BM, BN>::kChunksW) {
            const int64_t rw = min(n0 + row, n - 1);
            t.w[i] = kk < k ? *reinterpret_cast<const i32x4 *>(w + rw * k + kk) : i32x4{0, 0, 0, 0};
        }
        if (i < Tile<BM, BN>::kChunksA) {
            const int64_t ra = min(m0 + row, m - 1);
            t.a[i] = kk < k ? *reinterpret_cast<const i32x4 *>(a + ra * k + kk) : i32x4{0, 0, 0, 0};
        }
    }
}

template <int BM, int BN>
__device__ __forceinline__ void store_tiles(const TileLoad<BM, BN> &t, int8_t *lds_a, int8_t *lds_w, int tid) {
#pragma unroll
    for (int i = 0; i < Tile<BM, BN>::kChunks; ++i) {
        const int id = tid + kThreads * i;
        const int row = id >> 3;
        const int chunk = id & 7;
        if (i < Tile<BM, BN>::kChunksW) *reinterpret_cast<i32x4 *>(lds_w + swz(row, chunk)) = t.w[i];
        if (i < Tile<BM, BN>::kChunksA) *reinterpret_cast<i32x4 *>(lds_a + swz(row, chunk)) = t.a[i];
    }
}

// Linear tile index t -> (m-tile, n-tile): groups of kGroupM m-tiles,
// m-major inside a group.
__device__ __forceinline__ void tile_of(int t, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gsm = min(tiles_m - first_m, kGroupM);
    const int in_group = t % per_group;
    tm = first_m + in_group % gsm;
    tn = in_group / gsm;
}

// Maps the linear workgroup id to (m-tile, n-tile): XCD x (workgroup id mod
// 8) owns a contiguous range of tile indices, walked in order.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int total = tiles_m * tiles_n;
    const int q = total / 8, r = total % 8;
    const int xcd = bid % 8, idx = bid / 8;
    const int t = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
    tile_of(t, tiles_m, tiles_n, tm, tn);
}

constexpr int kStages = 2;
typedef __attribute__((address_space(3))) void lds_void;

// Per-lane source offsets of the direct-to-LDS loads.  Wave w fills the 1 KiB
// blocks w * kABlocks .. of the activation panel and w * kWBlocks .. of the
// weight panel; in block b, lane l writes LDS row 8 b + l / 8, physical chunk
// l % 8, which holds logical chunk (l % 8) ^ ((row >> 1) & 7) of that row.
// Offsets are relative to the panel's first row at K offset 0 (32-bit: a
// panel row index times K plus a chunk offset; rows past the end are
// clamped, their results never stored).
template <int BM, int BN>
struct LoadGeom {
    uint32_t a_off[Tile<BM, BN>::kABlocks];
    uint32_t w_off[Tile<BM, BN>::kWBlocks];
};

template <int BM, int BN>
__device__ __forceinline__ LoadGeom<BM, BN> load_geom(int64_t m0, int64_t n0, int64_t m, int64_t n, int64_t k,
                                                      int wave, int lane) {
    LoadGeom<BM, BN> gm;
#pragma unroll
    for (int i = 0; i < Tile<BM, BN>::kABlocks; ++i) {
        const int row = 8 * (Tile<BM, BN>::kABlocks * wave + i) + (lane >> 3);
        const int c = (lane & 7) ^ ((row >> 1) & 7);
        gm.a_off[i] = static_cast<uint32_t>((min(m0 + row, m - 1) - m0) * k + c * 16);
    }
#pragma unroll
    for (int i = 0; i < Tile<BM, BN>::kWBlocks; ++i) {
        const int row = 8 * (Tile<BM, BN>::kWBlocks * wave + i) + (lane >> 3);
        const int c = (lane & 7) ^ ((row >> 1) & 7);
        gm.w_off[i] = static_cast<uint32_t>((min(n0 + row, n - 1) - n0) * k + c * 16);
    }
    return gm;
}

// A pointer that is the same in every lane, rebuilt from readfirstlane of
// its two halves.
__device__ __forceinline__ const int8_t *uniform_ptr(const int8_t *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<const int8_t *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Direct-to-LDS loads of one full K step into a ring stage: buffer loads with
// the lane's 32-bit offset within the panel and the step's K offset k0 as
// the scalar offset, so no 64-bit address is formed per load.
// One overload per tile height: the host compilation pass rejects a template
// of this function (the buffer builtins exist only for the device target).
#define TU_ISSUE_STEP_BODY(BM, BN)                                                                               \
    _Pragma("unroll") for (int i = 0; i < Tile<BM, BN>::kBlocks; ++i) {                                         \
        if (i < Tile<BM, BN>::kABlocks)                                                                         \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(                                                           \
                ars, (lds_void *)(stage + (Tile<BM, BN>::kABlocks * wave + i) * 1024), 16, gm.a_off[i], k0, 0, 0); \
        if (i < Tile<BM, BN>::kWBlocks)                                                                         \
            __builtin_amdgcn_raw_ptr_buffer_load_lds(                                                           \
                wrs, (lds_void *)(stage + BM * kBK + (Tile<BM, BN>::kWBlocks * wave + i) * 1024), 16, gm.w_off[i], \
                k0, 0, 0);                                                                                      \
    }
__device__ __forceinline__ void issue_step(int8_t *stage, __amdgpu_buffer_rsrc_t ars, __amdgpu_buffer_rsrc_t wrs,
                                           const LoadGeom<256, 256> &gm, uint32_t k0, int wave) {
    TU_ISSUE_STEP_BODY(256, 256)
}
__device__ __forceinline__ void issue_step(int8_t *stage, __amdgpu_buffer_rsrc_t ars, __amdgpu_buffer_rsrc_t wrs,
                                           const LoadGeom<128, 256> &gm, uint32_t k0, int wave) {
    TU_ISSUE_STEP_BODY(128, 256)
}
__device__ __forceinline__ void issue_step(int8_t *stage, __amdgpu_buffer_rsrc_t ars, __amdgpu_buffer_rsrc_t wrs,
                                           const LoadGeom<256, 192> &gm, uint32_t k0, int wave) {
    TU_ISSUE_STEP_BODY(256, 192)
}
#undef TU_ISSUE_STEP_BODY

template <int BM, int BN>
struct Frags {
    i32x4 a[Tile<BM, BN>::kFragsN];  // weight rows (MFMA A operand)
    i32x4 b[Tile<BM, BN>::kFragsM];  // activation rows (MFMA B operand)
};

// (1, 1) in bf16: the gate of a residual add without one.
constexpr uint32_t kBf16OnePair = 0x3f803f80u;

// Output kinds of the kernel's epilogue.
constexpr int kOutBf16 = 0;  // bf16_rn of the fp32 epilogue value (LDS-staged row stores)
constexpr int kOutF16 = 1;   // fp16_rn of the same value (LDS-staged row stores)
constexpr int kOutF32 = 2;   // the fp32 value itself (direct 16-byte stores)
constexpr int kOutI32 = 3;   // the int32 accumulator (direct 16-byte stores)

// kResidual: out = bf16_rn(fma(y, gate[row / gate_rows][col], residual[row][col]))
// with y the bf16 epilogue value (gate 1 when absent).  residual may be out
// (in place), so neither carries __restrict__: each output chunk is read as
// residual and then written by the same lane, and no lane stores a chunk
// that another lane reads (clamped reads past the last row feed only rows
// that are never stored).
template <int BM, int BN, int kOut, bool kResidual>
__global__ __launch_bounds__(kThreads, kWaves / 4) void int8_gemm_kernel(
    const int8_t *__restrict__ a, const int8_t *__restrict__ w, const float *__restrict__ as,
    const float *__restrict__ ws, const float *__restrict__ bias, void *out,
    int64_t m, int64_t n, int64_t k, int tiles_m, int tiles_n, const uint16_t *residual, const uint16_t *gate,
    int64_t gate_rows) {
    constexpr int kBM = BM;
    constexpr int kFragsM = Tile<BM, BN>::kFragsM;
    constexpr int kFragsN = Tile<BM, BN>::kFragsN;
    constexpr int kStageBytes = Tile<BM, BN>::kStageBytes;
    __shared__ __align__(1024) int8_t lds_mem[Tile<BM, BN>::kLdsBytes];
    auto lds = [&](int st) { return lds_mem + st * kStageBytes; };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave / kWavesM;  // which half (BN / 2 rows) of the W tile
    const int wm = wave % kWavesM;  // which activation-row slice of the tile

    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    // Uniform by construction; said explicitly so the panel buffer resources
    // are formed in scalar registers.
    tm = __builtin_amdgcn_readfirstlane(tm);
    tn = __builtin_amdgcn_readfirstlane(tn);
    const int64_t m0 = static_cast<int64_t>(tm) * kBM;
    const int64_t n0 = static_cast<int64_t>(tn) * BN;
    const LoadGeom<BM, BN> gm = load_geom<BM, BN>(m0, n0, m, n, k, wave, lane);
    // Buffer resources over the tile's two panels (BM and 256 rows of K bytes,
    // K < 2^17, so every offset fits in 32 bits).  The panel addresses are
    // uniform; passing them through readfirstlane keeps the resources in
    // scalar registers.
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(uniform_ptr(a + m0 * k), static_cast<uint32_t>(kBM * k));
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(uniform_ptr(w + n0 * k), static_cast<uint32_t>(BN * k));

    i32x4 acc[kFragsN][kFragsM];
#pragma unroll
    for (int i = 0; i < kFragsN; ++i)
#pragma unroll
        for (int j = 0; j < kFragsM; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    const int frag_row = lane & 15;
    const int frag_chunk = lane >> 4;
    // Fragments of 64-deep slice kk (0 or 1) of a stage.
    auto load_frags = [&](Frags<BM, BN> &f, const int8_t *stage, int kk) {
        const int8_t *la = stage;
        const int8_t *lw = stage + kBM * kBK;
#pragma unroll
        for (int j = 0; j < kFragsM; ++j)
            f.b[j] = *reinterpret_cast<const i32x4 *>(
                la + swz(wm * 16 * kFragsM + j * 16 + frag_row, 4 * kk + frag_chunk));
#pragma unroll
        for (int i = 0; i < kFragsN; ++i)
            f.a[i] = *reinterpret_cast<const i32x4 *>(lw + swz(wn * (BN / 2) + i * 16 + frag_row, 4 * kk + frag_chunk));
    };
    // A slice's MFMAs walk the (i, j) fragment grid as a snake: j runs up on
    // even i and down on odd i, so consecutive MFMAs always share one operand
    // (at a row change the activation fragment stays).  Under the board power
    // limit the fewer operand changes measured 0.5-1 % faster at the Wan
    // shapes; each accumulator's K order, and so every result, is unchanged.
    auto mma = [&](const Frags<BM, BN> &f) {
#pragma unroll
        for (int i = 0; i < kFragsN; ++i)
#pragma unroll
            for (int jj = 0; jj < kFragsM; ++jj) {
                const int j = (i & 1) ? kFragsM - 1 - jj : jj;
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
            }
    };
    // MFMAs [b, e) of a slice in the same order; b and e are constants at
    // every call, so the loop unrolls to fixed accumulator registers.
    auto mma_part = [&](const Frags<BM, BN> &f, int b, int e) {
#pragma unroll
        for (int x = b; x < e; ++x) {
            const int i = x / kFragsM;
            const int j = (i & 1) ? kFragsM - 1 - x % kFragsM : x % kFragsM;
            acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
        }
    };

    const int full = static_cast<int>(k / kBK);
    if (full > 0) {
        issue_step(lds(0), ars, wrs, gm, 0, wave);
        if (full > 1) issue_step(lds(1), ars, wrs, gm, kBK, wave);
        if (full > 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(Tile<BM, BN>::kLoads));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        Frags<BM, BN> f0, f1;
        load_frags(f0, lds(0), 0);
        __builtin_amdgcn_s_waitcnt(lgkmcnt_imm(0));
        // One K step:
        //   slice 1 reads, with the first kPre MFMAs of slice 0 covering them
        //   barrier: step s + 1 resident, every wave done reading stage s
        //   rest of slice 0, interleaved with the loads of step s + 2
        //   slice 1, interleaved with the reads of slice 0 of step s + 1
        // so the MFMA pipe has work on both sides of the barrier.  Slice 0's
        // fragments are in registers when a step starts (their reads retire
        // at the end of the previous step), so only 12 LDS reads are ever in
        // flight and no MFMA waits on one (with more than 15 in flight the
        // compiler can only wait for all of them).  The loop body has no
        // branches, which the register allocation needs: the last two steps
        // load step full - 1 again into stages nobody reads any more, and
        // those loads are retired after the loop, before the ring is reused.
        constexpr int kMma = Tile<BM, BN>::kMma, kPre = Tile<BM, BN>::kPre;
#pragma clang loop unroll(disable)
        for (int s = 0; s < full; ++s) {
            const uint32_t k2 = static_cast<uint32_t>(min(s + 2, full - 1) * kBK);
            load_frags(f1, lds(s & 1), 1);
            mma_part(f0, 0, kPre);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            issue_step(lds(s & 1), ars, wrs, gm, k2, wave);
            mma_part(f0, kPre, kMma);
#pragma unroll
            for (int i = 0; i < Tile<BM, BN>::kLoads; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_frags(f0, lds((s + 1) & 1), 0);
            mma(f1);
#pragma unroll
            for (int i = 0; i < kFragsN + kFragsM; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(lgkmcnt_imm(0));
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    if (full * kBK < k) {
        // Partial last step: register loads with zero fill past K.
        __syncthreads();
        TileLoad<BM, BN> t;
        load_tiles<BM, BN>(t, a, w, m0, n0, m, n, k, static_cast<int64_t>(full) * kBK, tid);
        store_tiles<BM, BN>(t, lds(0), lds(0) + kBM * kBK, tid);
        __syncthreads();
        Frags<BM, BN> f;
        load_frags(f, lds(0), 0);
        mma(f);
        load_frags(f, lds(0), 1);
        mma(f);
    }

    // acc[i][j][r] = C[m = m0 + wm*16*kFragsM + 16j + (lane & 15)]
    //                  [n = n0 + wn*BN/2 + 16i + 4*(lane >> 4) + r]
    const int g = lane >> 4;
    if constexpr (kOut == kOutI32) {
#pragma unroll
        for (int j = 0; j < kFragsM; ++j) {
            const int64_t row = m0 + wm * 16 * kFragsM + j * 16 + (lane & 15);
            if (row >= m) continue;
#pragma unroll
            for (int i = 0; i < kFragsN; ++i) {
                const int64_t col = n0 + wn * (BN / 2) + i * 16 + 4 * g;
                if (col >= n) continue;  // n % 8 == 0, so a group of 4 is all in or all out
                __builtin_nontemporal_store(acc[i][j], reinterpret_cast<i32x4 *>(static_cast<int32_t *>(out) + row * n + col));
            }
        }
    } else if constexpr (kOut == kOutF32) {
        // fp32 values straight from the accumulators: each lane holds 4
        // consecutive columns of one row, one 16-byte store per 16 x 16 block
        // (no rounding, so no staging for row-wide stores either).
        const float *bp = bias ? bias : ws;
#pragma unroll
        for (int j = 0; j < kFragsM; ++j) {
            const int64_t row = m0 + wm * 16 * kFragsM + j * 16 + (lane & 15);
            const float xs = as[min(row, m - 1)];
#pragma unroll
            for (int i = 0; i < kFragsN; ++i) {
                const int64_t col = n0 + wn * (BN / 2) + i * 16 + 4 * g;
                const int64_t cc = min(col, n - 4);
                const f32x4 wsv = *reinterpret_cast<const f32x4 *>(ws + cc);
                const f32x4 bv = *reinterpret_cast<const f32x4 *>(bp + cc);
                f32x4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = static_cast<float>(acc[i][j][r]);
                    x = x * xs;
                    x = x * wsv[r];
                    if (bias) x = x + bv[r];
                    v[r] = x;
                }
                if (row < m && col < n)  // n % 8 == 0: a group of 4 is all in or all out
                    __builtin_nontemporal_store(v, reinterpret_cast<f32x4 *>(static_cast<float *>(out) + row * n + col));
            }
        }
    } else {
        // 16-bit tile of this wave (16 kFragsM rows x 128 columns) staged
        // through LDS, so that global stores write whole rows: the ring is
        // free once every wave is past its last fragment read.  Rows of 256 B;
        // the 16-byte chunk index is XORed with the row's low 4 bits (both the
        // 8-byte writes below and the 16-byte row reads are conflict free).
        static_assert(kOut == kOutBf16 || !kResidual, "the residual epilogue writes bf16");
        constexpr int kRows = 16 * kFragsM;
        const int frow = lane & 15;
        const int64_t row_base = m0 + wm * kRows;
        const int64_t col_base = n0 + wn * (BN / 2);
        // All of the tile's scales and bias in one batch, from in-range
        // addresses without branches (rows / columns past the end read the
        // last valid ones and are never stored): vector-memory operations
        // retire in order, so loads interleaved with their uses would each
        // wait a full round trip.
        const float *bp = bias ? bias : ws;
        float arow[kFragsM];
        f32x4 wsv[kFragsN], bv[kFragsN];
#pragma unroll
        for (int j = 0; j < kFragsM; ++j) arow[j] = as[min(row_base + j * 16 + frow, m - 1)];
#pragma unroll
        for (int i = 0; i < kFragsN; ++i) {
            const int64_t col = min(col_base + i * 16 + 4 * g, n - 4);
            wsv[i] = *reinterpret_cast<const f32x4 *>(ws + col);
            bv[i] = *reinterpret_cast<const f32x4 *>(bp + col);
        }
        // With finite row scales and bias and finite nonzero column scales no
        // value of the wave's tile can be NaN: float(acc) is finite, a product
        // or sum of finite values overflows at most to +-inf, and +-inf times
        // a nonzero scale plus a finite bias stays +-inf.  The hardware RNE
        // conversion then equals bf16_rne_bits bit for bit, at one
        // instruction per pair instead of about five per value; any other
        // wave takes the software rounding (canonical 0x7fff NaN), and so does
        // the residual variant, which has no registers to spare for both.
        uint32_t finite_max = 0, ws_max = 0;
#pragma unroll
        for (int j = 0; j < kFragsM; ++j) finite_max = max(finite_max, __float_as_uint(arow[j]) & 0x7fffffffu);
#pragma unroll
        for (int i = 0; i < kFragsN; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                finite_max = max(finite_max, __float_as_uint(bv[i][r]) & 0x7fffffffu);
                // |ws| bits - 1 (unsigned): 0 wraps to 0xffffffff
                ws_max = max(ws_max, (__float_as_uint(wsv[i][r]) & 0x7fffffffu) - 1u);
            }
        const bool hw_round = !kResidual &&
            __builtin_amdgcn_ballot_w64(finite_max >= 0x7f800000u || ws_max >= 0x7f7fffffu) == 0;
        __syncthreads();
        int8_t *tile = lds_mem + wave * kRows * 256;
        auto stage_tile = [&](auto hw) {
#pragma unroll
            for (int j = 0; j < kFragsM; ++j) {
                const int lrow = j * 16 + frow;
#pragma unroll
                for (int i = 0; i < kFragsN; ++i) {
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = static_cast<float>(acc[i][j][r]);
                        x = x * arow[j];
                        x = x * wsv[i][r];
                        if (bias) x = x + bv[i][r];
                        v[r] = x;
                    }
                    u32x2 packed;
                    if constexpr (kOut == kOutF16) {
                        // RNE by the hardware conversion; only the slow path
                        // can meet a NaN, which it writes as 0x7e00
                        if constexpr (decltype(hw)::value) {
                            packed.x = hw_f16x2_bits(v[0], v[1]);
                            packed.y = hw_f16x2_bits(v[2], v[3]);
                        } else {
                            packed.x = pack_f16x2(v[0], v[1]);
                            packed.y = pack_f16x2(v[2], v[3]);
                        }
                    } else if constexpr (decltype(hw)::value) {
                        packed.x = hw_bf16x2_bits(v[0], v[1]);
                        packed.y = hw_bf16x2_bits(v[2], v[3]);
                    } else {
                        packed.x = pack_bf16x2(v[0], v[1]);
                        packed.y = pack_bf16x2(v[2], v[3]);
                    }
                    const int chunk = (2 * i + (g >> 1)) ^ (lrow & 15);
                    *reinterpret_cast<u32x2 *>(tile + lrow * 256 + chunk * 16 + (g & 1) * 8) = packed;
                }
            }
        };
        if (hw_round) stage_tile(std::true_type{});
        else stage_tile(std::false_type{});
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // 4 rows of 16 chunks per pass (a wave's BN / 2 columns are the
        // first BN / 16 chunks of a row)
        const int rsub = lane >> 4, c = lane & 15;
        // residual (and gate) chunks of every pass, loaded before any store
        u32x4 res[kResidual ? kRows / 4 : 1], gv[kResidual ? kRows / 4 : 1];
        if constexpr (kResidual) {
#pragma unroll
            for (int pass = 0; pass < kRows / 4; ++pass) {
                const int64_t row = min(row_base + pass * 4 + rsub, m - 1);
                const int64_t col = min(col_base + c * 8, n - 8);
                res[pass] = *reinterpret_cast<const u32x4 *>(residual + row * n + col);
                gv[pass] = gate ? *reinterpret_cast<const u32x4 *>(gate + (row / gate_rows) * n + col)
                                : u32x4{kBf16OnePair, kBf16OnePair, kBf16OnePair, kBf16OnePair};
            }
        }
#pragma unroll
        for (int pass = 0; pass < kRows / 4; ++pass) {
            const int lrow = pass * 4 + rsub;
            const int64_t row = row_base + lrow;
            const int64_t col = col_base + c * 8;
            u32x4 val = *reinterpret_cast<const u32x4 *>(tile + lrow * 256 + ((c ^ (lrow & 15)) << 4));
            if constexpr (kResidual) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t y = val[e], r = res[pass][e], gg = gv[pass][e];
                    const float lo = __builtin_fmaf(__uint_as_float(y << 16), __uint_as_float(gg << 16),
                                                    __uint_as_float(r << 16));
                    const float hi = __builtin_fmaf(__uint_as_float(y & 0xffff0000u), __uint_as_float(gg & 0xffff0000u),
                                                    __uint_as_float(r & 0xffff0000u));
                    val[e] = pack_bf16x2(lo, hi);
                }
            }
            if (row < m && col < n && c < BN / 16)  // n % 8 == 0: a chunk is all in or all out
                __builtin_nontemporal_store(val, reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(out) + row * n + col));
        }
    }
}

// out[m][c] = bf16_rn((float(acc[m*ld + c]) * as[m]) * ws[c or 0]),
// bf16_epilogue.cu:46-143.  Each thread converts 4 consecutive columns when
// the row width allows, else one.
template <bool kScalarWs, bool kVec4>
__global__ __launch_bounds__(256) void dequant_kernel(const int32_t *__restrict__ acc, int64_t ld,
                                                      const float *__restrict__ as,
                                                      const float *__restrict__ ws,
                                                      uint16_t *__restrict__ out, int64_t m,
                                                      int64_t cols) {
    const int64_t per_row = kVec4 ? cols / 4 : cols;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= m * per_row) return;
    const int64_t row = idx / per_row;
    const int64_t c = (idx - row * per_row) * (kVec4 ? 4 : 1);
    const float xs = as[row];
    if constexpr (kVec4) {
        const i32x4 v = *reinterpret_cast<const i32x4 *>(acc + row * ld + c);
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = (static_cast<float>(v[e]) * xs) * ws[kScalarWs ? 0 : c + e];
        u32x2 p;
        p.x = pack_bf16x2(r[0], r[1]);
        p.y = pack_bf16x2(r[2], r[3]);
        *reinterpret_cast<u32x2 *>(out + row * cols + c) = p;
    } else {
        const float r = (static_cast<float>(acc[row * ld + c]) * xs) * ws[kScalarWs ? 0 : c];
        out[row * cols + c] = static_cast<uint16_t>(bf16_rne_bits(r));
    }
}

int32_t check_gemm_args(const int8_t *a, const int8_t *w, const void *out, int64_t m, int64_t n,
                        int64_t k) {
    TU_REQUIRE(m >= 0 && n > 0 && k > 0, "INT8 GEMM dimensions must be positive (m=%lld n=%lld k=%lld)",
               static_cast<long long>(m), static_cast<long long>(n), static_cast<long long>(k));
    TU_REQUIRE(k % 16 == 0 && n % 8 == 0, "INT8 GEMM requires K%%16==0 and N%%8==0 (K=%lld N=%lld)",
               static_cast<long long>(k), static_cast<long long>(n));
    TU_REQUIRE(k < 131072, "INT8 GEMM K=%lld would overflow the int32 accumulator", static_cast<long long>(k));
    TU_REQUIRE((m + 127) / 128 * ((n + 191) / 192) < 0x7fffffff, "INT8 GEMM grid too large");
    TU_REQUIRE(a && w && out, "INT8 GEMM pointers must be non-null");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0,
               "INT8 GEMM operands must be 16-byte aligned");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0, "INT8 GEMM output must be 16-byte aligned");
    return require_gfx950();
}

// Time of a round of 128-row tiles relative to a round of 256-row tiles of the
// same N and K, measured on MI355X: 0.635 at N 8960 / K 1536 and at N 5120 /
// K 5120 (a tile's fixed part, the epilogue's stores and the first loads, does
// not halve with its rows).
constexpr double kHalfTileCost = TU_GEMM_HALF_TILE_COST;
// The same for a round of 256 x 192 tiles: 0.83-0.88 measured at K 1536 and
// K 5120 (0.75 of the MFMAs plus the fixed part).
constexpr double kTile192Cost = 0.85;

// Tile policy from the grid: one workgroup per CU, so tiles run in rounds of
// `cus`; 128 x 256 or 256 x 192 tiles are chosen when their rounds cost less
// than the 256 x 256 tiles' (a grid of a few, partly empty rounds).
int pick_tile_policy(int64_t m, int64_t n, int cus) {
    const int64_t t256 = (m + 255) / 256 * ((n + 255) / 256);
    const int64_t t128 = (m + 127) / 128 * ((n + 255) / 256);
    const int64_t t192 = (m + 255) / 256 * ((n + 191) / 192);
    const double c256 = static_cast<double>((t256 + cus - 1) / cus);
    const double c128 = static_cast<double>((t128 + cus - 1) / cus) * kHalfTileCost;
    const double c192 = static_cast<double>((t192 + cus - 1) / cus) * kTile192Cost;
    if (c128 < c256 && c128 <= c192) return TU_GEMM_TILE_128;
    if (c192 < c256) return TU_GEMM_TILE_192;
    return TU_GEMM_TILE_256;
}

template <int kOut, bool kResidual = false>
int32_t launch_gemm(const int8_t *a, const int8_t *w, const float *as, const float *ws, const float *bias,
                    void *out, int64_t m, int64_t n, int64_t k, void *stream, const uint16_t *residual = nullptr,
                    const uint16_t *gate = nullptr, int64_t gate_rows = 1, int policy = TU_GEMM_TILE_AUTO) {
    if (m == 0) return 0;
    if (policy == TU_GEMM_TILE_AUTO) {
        int cus = 0;
        if (device_cus(cus)) return -1;
        policy = pick_tile_policy(m, n, cus);
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (policy == TU_GEMM_TILE_128) {
        const int tiles_m = static_cast<int>((m + 127) / 128), tiles_n = static_cast<int>((n + 255) / 256);
        int8_gemm_kernel<128, 256, kOut, kResidual><<<dim3(tiles_m * tiles_n), kThreads, 0, st>>>(
            a, w, as, ws, bias, out, m, n, k, tiles_m, tiles_n, residual, gate, gate_rows);
    } else if (policy == TU_GEMM_TILE_192) {
        const int tiles_m = static_cast<int>((m + 255) / 256), tiles_n = static_cast<int>((n + 191) / 192);
        int8_gemm_kernel<256, 192, kOut, kResidual><<<dim3(tiles_m * tiles_n), kThreads, 0, st>>>(
            a, w, as, ws, bias, out, m, n, k, tiles_m, tiles_n, residual, gate, gate_rows);
    } else {
        const int tiles_m = static_cast<int>((m + 255) / 256), tiles_n = static_cast<int>((n + 255) / 256);
        int8_gemm_kernel<256, 256, kOut, kResidual><<<dim3(tiles_m * tiles_n), kThreads, 0, st>>>(
            a, w, as, ws, bias, out, m, n, k, tiles_m, tiles_n, residual, gate, gate_rows);
    }
    return check_launch(kOut == kOutI32   ? "tu_int8_gemm_i32"
                        : kResidual       ? "tu_int8_gemm_bf16_residual"
                        : kOut == kOutF16 ? "tu_int8_gemm_f16"
                        : kOut == kOutF32 ? "tu_int8_gemm_f32"
                                          : "tu_int8_gemm_bf16");
}

int32_t check_epilogue_args(const float *a_scale, const float *w_scale, const float *bias) {
    TU_REQUIRE(a_scale && w_scale, "INT8 GEMM scales must be non-null");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(w_scale) & 15) == 0 && (reinterpret_cast<uintptr_t>(bias) & 15) == 0,
               "INT8 GEMM weight scale and bias must be 16-byte aligned");
    return 0;
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_int8_gemm_bf16(const int8_t *a, const int8_t *w, const float *a_scale,
                                     const float *w_scale, const float *bias, void *out_bf16, int64_t m,
                                     int64_t n, int64_t k, void *stream) {
    using namespace tu;
    if (check_gemm_args(a, w, out_bf16, m, n, k) || check_epilogue_args(a_scale, w_scale, bias)) return -1;
    return launch_gemm<kOutBf16>(a, w, a_scale, w_scale, bias, out_bf16, m, n, k, stream);
}

extern "C" int32_t tu_int8_gemm_f16(const int8_t *a, const int8_t *w, const float *a_scale, const float *w_scale,
                                    const float *bias, void *out_f16, int64_t m, int64_t n, int64_t k,
                                    void *stream) {
    using namespace tu;
    if (check_gemm_args(a, w, out_f16, m, n, k) || check_epilogue_args(a_scale, w_scale, bias)) return -1;
    return launch_gemm<kOutF16>(a, w, a_scale, w_scale, bias, out_f16, m, n, k, stream);
}

extern "C" int32_t tu_int8_gemm_f32(const int8_t *a, const int8_t *w, const float *a_scale, const float *w_scale,
                                    const float *bias, float *out, int64_t m, int64_t n, int64_t k, void *stream) {
    using namespace tu;
    if (check_gemm_args(a, w, out, m, n, k) || check_epilogue_args(a_scale, w_scale, bias)) return -1;
    return launch_gemm<kOutF32>(a, w, a_scale, w_scale, bias, out, m, n, k, stream);
}

extern "C" int32_t tu_int8_gemm_bf16_residual(const int8_t *a, const int8_t *w, const float *a_scale,
                                              const float *w_scale, const float *bias, const void *residual_bf16,
                                              const void *gate_bf16, int64_t gate_rows, void *out_bf16, int64_t m,
                                              int64_t n, int64_t k, void *stream) {
    using namespace tu;
    if (check_gemm_args(a, w, out_bf16, m, n, k)) return -1;
    TU_REQUIRE(a_scale && w_scale && residual_bf16, "INT8 GEMM scales and residual must be non-null");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(w_scale) & 15) == 0 && (reinterpret_cast<uintptr_t>(bias) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(residual_bf16) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(gate_bf16) & 15) == 0,
               "INT8 GEMM weight scale, bias, residual and gate must be 16-byte aligned");
    TU_REQUIRE(!gate_bf16 || gate_rows > 0, "INT8 GEMM gate_rows must be positive with a gate (got %lld)",
               static_cast<long long>(gate_rows));
    return launch_gemm<kOutBf16, true>(a, w, a_scale, w_scale, bias, out_bf16, m, n, k, stream,
                                    static_cast<const uint16_t *>(residual_bf16),
                                    static_cast<const uint16_t *>(gate_bf16), gate_bf16 ? gate_rows : 1);
}

extern "C" int32_t tu_int8_gemm_i32(const int8_t *a, const int8_t *w, int32_t *acc, int64_t m, int64_t n,
                                    int64_t k, void *stream) {
    using namespace tu;
    if (check_gemm_args(a, w, acc, m, n, k)) return -1;
    return launch_gemm<kOutI32>(a, w, nullptr, nullptr, nullptr, acc, m, n, k, stream);
}

extern "C" int32_t tu_dequant_i32_bf16(const int32_t *acc, int64_t acc_ld, const float *a_scale,
                                       const float *w_scale, int32_t ws_scalar, void *out_bf16, int64_t m,
                                       int64_t cols, void *stream) {
    using namespace tu;
    TU_REQUIRE(m >= 0 && cols > 0 && acc_ld >= cols, "dequantize: need rows >= 0 and 0 < cols <= acc_ld");
    TU_REQUIRE(acc && a_scale && w_scale && out_bf16, "dequantize pointers must be non-null");
    if (require_gfx950()) return -1;
    if (m == 0) return 0;
    const bool vec4 = cols % 4 == 0 && acc_ld % 4 == 0 && (reinterpret_cast<uintptr_t>(acc) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(out_bf16) & 7) == 0;
    const int64_t work = m * (vec4 ? cols / 4 : cols);
    TU_REQUIRE((work + 255) / 256 < 0x7fffffff, "dequantize grid too large");
    const dim3 grid(static_cast<unsigned>((work + 255) / 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto *o = static_cast<uint16_t *>(out_bf16);
    if (ws_scalar) {
        if (vec4) dequant_kernel<true, true><<<grid, 256, 0, s>>>(acc, acc_ld, a_scale, w_scale, o, m, cols);
        else dequant_kernel<true, false><<<grid, 256, 0, s>>>(acc, acc_ld, a_scale, w_scale, o, m, cols);
    } else {
        if (vec4) dequant_kernel<false, true><<<grid, 256, 0, s>>>(acc, acc_ld, a_scale, w_scale, o, m, cols);
        else dequant_kernel<false, false><<<grid, 256, 0, s>>>(acc, acc_ld, a_scale, w_scale, o, m, cols);
    }
    return check_launch("tu_dequant_i32_bf16");
}

extern "C" int32_t tu_int8_gemm_ex(const int8_t *a, const int8_t *w, const float *a_scale, const float *w_scale,
                                   const float *bias, void *out, int32_t out_type, int64_t m, int64_t n, int64_t k,
                                   int32_t tile_policy, void *stream) {
    using namespace tu;
    TU_REQUIRE(tile_policy == TU_GEMM_TILE_AUTO || tile_policy == TU_GEMM_TILE_256 || tile_policy == TU_GEMM_TILE_128 ||
                   tile_policy == TU_GEMM_TILE_192,
               "INT8 GEMM tile_policy must be 0 (auto), 1 (256 x 256), 2 (128 x 256) or 3 (256 x 192), got %d",
               tile_policy);
    if (check_gemm_args(a, w, out, m, n, k)) return -1;
    switch (out_type) {
    case TU_OUT_I32:
        return launch_gemm<kOutI32>(a, w, nullptr, nullptr, nullptr, out, m, n, k, stream, nullptr, nullptr, 1,
                                    tile_policy);
    case TU_OUT_BF16:
        if (check_epilogue_args(a_scale, w_scale, bias)) return -1;
        return launch_gemm<kOutBf16>(a, w, a_scale, w_scale, bias, out, m, n, k, stream, nullptr, nullptr, 1,
                                     tile_policy);
    case TU_OUT_F16:
        if (check_epilogue_args(a_scale, w_scale, bias)) return -1;
        return launch_gemm<kOutF16>(a, w, a_scale, w_scale, bias, out, m, n, k, stream, nullptr, nullptr, 1,
                                    tile_policy);
    case TU_OUT_F32:
        if (check_epilogue_args(a_scale, w_scale, bias)) return -1;
        return launch_gemm<kOutF32>(a, w, a_scale, w_scale, bias, out, m, n, k, stream, nullptr, nullptr, 1,
                                    tile_policy);
    default:
        return fail("INT8 GEMM out_type must be 0 (bf16), 1 (fp16), 2 (fp32) or 3 (int32), got %d", out_type);
    }
}

extern "C" int32_t tu_int8_gemm_tile_policy(int64_t m, int64_t n, int32_t cus) {
    if (m <= 0 || n <= 0 || cus <= 0) return TU_GEMM_TILE_256;
    return tu::pick_tile_policy(m, n, cus);
}
