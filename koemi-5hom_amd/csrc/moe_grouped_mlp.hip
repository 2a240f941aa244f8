// Grouped expert GLU feed-forward for gfx950.
//
// Reference: cuda_kernels/moe/moe_kernels.cu:147-199, 501-558 — one block per
// sorted pair computing W_o (silu(W_g x + b_g) * (W_v x + b_v)) + b_o with
// scalar FMAs, re-reading the expert's weights for every pair. Here each
// expert's rows form a dense GEMM segment and the work runs as two grouped
// GEMMs on bf16 MFMA (v_mfma_f32_32x32x16_bf16, fp32 accumulation):
//
//   GEMM 1: H[rows_e, hidden] = glu(X_e W_g[e]^T + b_g, X_e W_v[e]^T + b_v),
//           one B tile holds 64 gate rows and the 64 value rows of the same
//           hidden units, so the SiLU-GLU product is formed in registers and H
//           is written once (bf16);
//   GEMM 2: Y[rows_e, width] = H W_o[e]^T + b_o.
//
// Both operands are K-contiguous ("TN"), so every MFMA fragment is one 16-byte
// LDS read per lane. The tile schedule is built on device from segment_offsets
// (no host synchronisation): tile slot -> (expert, first row). Rows past the
// valid pairs are zero-filled.
#include "common.hpp"
#include "mfma_stage.hpp"

#include <type_traits>

namespace koemi {
namespace {

using mfma_stage::bf16x8;
using mfma_stage::f32x16;
using mfma_stage::kOperandBytes;
using mfma_stage::slot_swizzle;
using mfma_stage::TileShape;
using mfma_stage::uniform_ptr;

// Block tile 256 (pairs) x BNT (B rows), the main loop of mfma_stage.hpp.
// Two tile shapes. BNT = 256: a 256 x 256 tile, 256 accumulators per wave and
// a ring of four 32 KiB stages (128 KiB of LDS), one workgroup per CU. BNT =
// 128: a 256 x 128 tile, 128 accumulators per wave and three 24 KiB stages
// (72 KiB), so that two workgroups share a CU and one's epilogue, prologue and
// memory waits overlap the other's matrix work.
constexpr int kBM = mfma_stage::kBM;
constexpr int kBN = 256;
constexpr int kBK = mfma_stage::kBK;
constexpr int kGemmThreads = mfma_stage::kThreads;
constexpr int kGroupM = 4;  // tile slots per group in the launch order (2 and 8 measured no better)
#ifndef KOEMI_GEMM_BN
#define KOEMI_GEMM_BN 256
#endif
// Rows are 64 bytes; the K step of the fronts' MFMA shape check.
constexpr int kKAlign = 64;

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Split K for the last, sparse round: at most this many partial tiles (fp32,
// at most 256 x 256 each, 64 MiB in all) per GEMM launch.
constexpr int kMaxSplitUnits = 256;
constexpr int kMaxSplit = 4;  // chunks per leftover tile (the fixup reads every chunk)
constexpr size_t kPartialTileFloats = static_cast<size_t>(kBM) * kBN;  // the workspace's room per partial tile

struct MlpWorkspace {
    size_t hidden_off, slot_expert_off, slot_row_off, slot_end_off, partial_off, total;
    int64_t max_slots;
};

// The MFMA path (both GEMM K dimensions multiples of kKAlign) keeps H in bf16; the
// SIMT path keeps it in fp32.
inline bool mfma_shape(int64_t width, int64_t hidden, int dtype) {
    return dtype == KOEMI_BF16 && width % kKAlign == 0 && hidden % kKAlign == 0;
}

inline MlpWorkspace mlp_workspace(int64_t pairs, int64_t width, int64_t hidden, int64_t E, int dtype) {
    MlpWorkspace w;
    w.max_slots = (pairs + kBM - 1) / kBM + E;
    const size_t elem = mfma_shape(width, hidden, dtype) ? 2 : 4;
    w.hidden_off = 0;
    w.slot_expert_off = align256(static_cast<size_t>(pairs > 0 ? pairs : 1) * static_cast<size_t>(hidden) * elem);
    // slot_expert has one more entry: the number of slots in use.
    w.slot_row_off = w.slot_expert_off + align256(static_cast<size_t>(w.max_slots + 1) * sizeof(int32_t));
    w.slot_end_off = w.slot_row_off + align256(static_cast<size_t>(w.max_slots) * sizeof(int64_t));
    w.partial_off = w.slot_end_off + align256(static_cast<size_t>(w.max_slots) * sizeof(int64_t));
    w.total = w.partial_off;
    if (mfma_shape(width, hidden, dtype)) w.total += kMaxSplitUnits * kPartialTileFloats * sizeof(float);
    return w;
}

__device__ __forceinline__ float silu_f(float v) {
    const float e = __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// slot -> (expert, first row, segment end) for every BM-row tile of every
// expert segment, built by one workgroup: per-expert tile counts, their
// exclusive prefix in LDS, then a binary search per slot. Segment bounds are
// clamped to [0, pairs] so that malformed offsets can never address rows
// outside the operands.
constexpr int kSchedThreads = 1024;
constexpr int64_t kMaxScheduleExperts = 8191;  // (E + 1) int32 tile prefixes stay within 32 KiB of LDS

__device__ __forceinline__ void segment_bounds(const int64_t* __restrict__ offsets, int64_t e, int64_t pairs,
                                               int64_t& lo, int64_t& hi) {
    lo = min(max(offsets[e], int64_t(0)), pairs);
    hi = min(max(offsets[e + 1], lo), pairs);
}

__global__ __launch_bounds__(kSchedThreads) void build_schedule_kernel(
    const int64_t* __restrict__ offsets, int64_t E, int64_t pairs, int64_t max_slots,
    int32_t* __restrict__ slot_expert, int64_t* __restrict__ slot_row, int64_t* __restrict__ slot_end) {
    extern __shared__ int32_t first_tile[];  // E + 1 entries
    __shared__ int32_t wave_tot[kSchedThreads / kWave];
    const int tid = threadIdx.x;
    const int64_t n = E + 1;
    for (int64_t e = tid; e < E; e += kSchedThreads) {
        int64_t lo, hi;
        segment_bounds(offsets, e, pairs, lo, hi);
        first_tile[e] = static_cast<int32_t>((hi - lo + kBM - 1) / kBM);
    }
    if (tid == 0) first_tile[E] = 0;
    __syncthreads();
    const int64_t per = (n + kSchedThreads - 1) / kSchedThreads;
    const int64_t b0 = min(n, tid * per), b1 = min(n, b0 + per);
    int32_t sum = 0;
    for (int64_t e = b0; e < b1; ++e) sum += first_tile[e];
    int32_t total_tiles;
    int32_t run = block_exclusive_scan<kSchedThreads>(sum, wave_tot, total_tiles);
    for (int64_t e = b0; e < b1; ++e) {
        const int32_t v = first_tile[e];
        first_tile[e] = run;
        run += v;
    }
    __syncthreads();
    const int64_t total = first_tile[E];
    if (tid == 0) slot_expert[max_slots] = static_cast<int32_t>(total);  // slots in use
    for (int64_t slot = tid; slot < max_slots; slot += kSchedThreads) {
        if (slot >= total) {
            slot_expert[slot] = -1;
            slot_row[slot] = 0;
            slot_end[slot] = 0;
            continue;
        }
        int64_t lo_e = 0, hi_e = E - 1;  // largest e with first_tile[e] <= slot
        while (lo_e < hi_e) {
            const int64_t mid = (lo_e + hi_e + 1) / 2;
            if (first_tile[mid] <= slot) lo_e = mid;
            else hi_e = mid - 1;
        }
        int64_t lo, hi;
        segment_bounds(offsets, lo_e, pairs, lo, hi);
        slot_expert[slot] = static_cast<int32_t>(lo_e);
        slot_row[slot] = lo + (slot - first_tile[lo_e]) * kBM;
        slot_end[slot] = hi;
    }
}

// Logical tile -> (slot, column tile): groups of kGroupM slots, all column
// tiles of a group before the next.
// Tile counts stay below 2^31 (the entry point checks), so the index
// arithmetic is 32-bit.
__device__ __forceinline__ void tile_coords(uint32_t logical, uint32_t slots, uint32_t n_tiles, uint32_t& slot,
                                            uint32_t& tile_n) {
    const uint32_t group = kGroupM * n_tiles;
    const uint32_t gi = logical / group;
    const uint32_t first_slot = gi * kGroupM;
    const uint32_t gm = min(static_cast<uint32_t>(kGroupM), slots - first_slot);
    const uint32_t within = logical - gi * group;
    slot = first_slot + within % gm;
    tile_n = within / gm;
}

// Work of one GEMM launch: `whole` tiles computed in full, then, when the tiles
// left over after whole rounds of `cus` workgroups (those that run at once)
// would fill at most a third of a round, each leftover tile split along K into
// `split` chunks, 3 or 4 (at least two K steps each), so that the last round
// keeps most CUs busy. Partial tiles go to the workspace as fp32 and a fixup
// kernel adds them in chunk order. (A two-way split measured slower than the
// half-empty round it replaces: its fp32 partials and the fix-up launch cost
// more than the half tile it saves. Up to eight chunks filled more CUs but
// wrote and re-read twice the fp32 partials: 11.7 against 7.9 us of fix-up
// per C5 layer, the partial tiles themselves unchanged.)
struct SplitPlan {
    uint32_t whole, units, split;
};

// float4 index of (wave, m-tile, n-tile, j, lane) in a partial tile of NT
// n-tiles per wave.
template <int NT>
__device__ __forceinline__ int partial_slot(int wave, int mt, int t, int j, int lane) {
    return (((wave * 4 + mt) * NT + t) * 4 + j) * kWave + lane;
}
__device__ __forceinline__ SplitPlan split_plan(uint32_t tiles, uint32_t nk, uint32_t cus) {
    SplitPlan p{tiles, 0, 1};
    const uint32_t rem = tiles % cus;
    if (rem > 0 && rem * 3 <= cus) {
        const uint32_t s =
            min(min(min(cus, static_cast<uint32_t>(kMaxSplitUnits)) / rem, nk / 2), static_cast<uint32_t>(kMaxSplit));
        if (s >= 3) {
            p.whole = tiles - rem;
            p.units = rem * s;
            p.split = s;
        }
    }
    return p;
}

// One 256 x BNT tile per workgroup. GLU: B rows 0 .. BNT/2 - 1 are gate rows
// and the next BNT/2 the value rows of hidden units [h0, h0 + BNT/2), so wave
// (wm, wn) holds gate and value accumulators of the same 128 rows x BNT/4
// hidden units and forms silu(g + b_g) * (u + b_v) in registers. Plain: BNT
// consecutive output columns, BNT/2 per wave. The MFMA is issued with the
// weight fragment as its first operand, so each lane's accumulators are four
// consecutive output columns of one row (8-byte stores). Launch order:
// workgroup i runs on XCD i % 8; tiles are renumbered so that every XCD owns a
// contiguous range, traversed in groups of kGroupM slots (all column tiles of
// a group before the next), which keeps the A rows and B columns of
// concurrently running tiles in that XCD's L2.
//
// gemm_tile is one tile: whole (PARTIAL false: all K steps, the epilogue) or
// a partial unit (K steps [k_begin, k_end), fp32 sums to the workspace); its
// two instances are inlined into separate branches of the kernel, so each
// keeps its own register allocation.
template <bool GLU, bool PARTIAL, int BNT>
__device__ __forceinline__ void gemm_tile(
    const bf16* __restrict__ A, const int64_t* __restrict__ a_index, int64_t a_count,
    const bf16* __restrict__ W0, const bf16* __restrict__ W1,
    const bf16* __restrict__ bias0, const bf16* __restrict__ bias1, bf16* __restrict__ C,
    const int32_t* __restrict__ slot_expert, const int64_t* __restrict__ slot_row,
    const int64_t* __restrict__ slot_end, int64_t n_out, int64_t K, int64_t n_tiles,
    float* __restrict__ partial, char* lds, float* bias_sh, uint32_t logical, uint32_t slots, uint32_t unit,
    uint32_t k_begin, uint32_t k_end) {
    using TS = TileShape<BNT>;
    constexpr int NT = TS::kNT;
    constexpr int kStages = TS::kStages;
    constexpr uint32_t kStageBytes = TS::kStageBytes;
    constexpr int CPT = TS::kCopies;
    uint32_t slot, tile_n;
    tile_coords(logical, slots, static_cast<uint32_t>(n_tiles), slot, tile_n);
    const int e = slot_expert[slot];
    if (e < 0) return;
    const int64_t row0 = slot_row[slot];
    const int64_t row_end = slot_end[slot];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t n0 = GLU ? static_cast<int64_t>(tile_n) * (BNT / 2) : static_cast<int64_t>(tile_n) * BNT;

    // Stage copies: A is 16 chunks of 1 KiB (16 rows each), wave w filling
    // chunks 4w .. 4w + 3; B is BNT / 16 chunks, wave w filling NT chunks from
    // NT w. Lane l of a chunk copies row l / 4 of it, K group (l % 4) ^
    // swizzle. Rows past the segment or the output width are clamped (they only
    // feed discarded outputs). Offsets are 32-bit and relative to per-tile
    // bases (the entry point bounds n_out * K; K * 256 is smaller). GLU: waves
    // 0-1 copy gate rows, waves 2-3 value rows. A partial tile runs K steps
    // [k_begin, k_end): the bases start there.
    // a_index (GEMM 1 reading the unsorted context): A row i of the tile is
    // context row a_index[row0 + i] (clamped to [0, a_count)), so the sorted
    // copy of the context is never built; the base is then the context itself.
    const int64_t k0 = static_cast<int64_t>(k_begin) * kBK;
    const bf16* a_base = static_cast<const bf16*>(uniform_ptr(A + (a_index ? 0 : row0 * K) + k0));
    const bf16* b_base = static_cast<const bf16*>(
        uniform_ptr(((GLU && wave >= 2) ? W1 : W0) + static_cast<int64_t>(e) * n_out * K + k0));
    const int a_rows = static_cast<int>(row_end - row0);
    uint32_t a_off[4], b_off[NT];  // byte offsets (the entry point bounds them below 2^32)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = (wave * 4 + i) * 16 + (lane >> 2);
        const int g = (lane & 3) ^ slot_swizzle(r);
        int64_t ar = min(r, a_rows - 1);
        if (a_index) ar = min(max(a_index[row0 + ar], int64_t(0)), a_count - 1);
        a_off[i] = (static_cast<uint32_t>(ar) * static_cast<uint32_t>(K) + g * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int r = (wave * NT + i) * 16 + (lane >> 2);
        const int g = (lane & 3) ^ slot_swizzle(r);
        const int64_t n = GLU ? min(n0 + (r & (BNT / 2 - 1)), n_out - 1) : min(n0 + r, n_out - 1);
        b_off[i] = (static_cast<uint32_t>(n) * static_cast<uint32_t>(K) + g * 8) * 2u;
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
    const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + wave * 4 * 1024);
    const uint32_t b_lds = __builtin_amdgcn_readfirstlane(lds0 + kOperandBytes + wave * NT * 1024);
    // Fragment rows: A rows of the wave's four m-tiles, B rows of its NT
    // n-tiles (GLU: NT / 2 gate, then NT / 2 value).
    const int fr = lane & 31;
    const int fg = lane >> 5;

    // The tile's biases (one per thread: GLU gate biases of hidden units
    // [n0, n0 + BNT/2) then their value biases; plain: BNT output columns;
    // threads past BNT load a clamped column nobody reads) are loaded now and
    // reach LDS at the epilogue, so their latency is hidden behind the main
    // loop.
    float bias_mine;
    {
        const int64_t col = GLU ? min(n0 + (tid & (BNT / 2 - 1)), n_out - 1) : min(n0 + min(tid, BNT - 1), n_out - 1);
        const bf16* bsrc = (GLU && (tid & (BNT - 1)) >= BNT / 2) ? bias1 : bias0;
        bias_mine = to_f32(bsrc[static_cast<int64_t>(e) * n_out + col]);
    }
    f32x16 acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    int a_row[4], b_row[NT];
#pragma unroll
    for (int t = 0; t < 4; ++t) a_row[t] = wm * 128 + t * 32 + fr;
#pragma unroll
    for (int t = 0; t < NT; ++t)
        b_row[t] = (GLU ? (t < NT / 2 ? wn * (BNT / 4) + t * 32 : BNT / 2 + wn * (BNT / 4) + (t - NT / 2) * 32)
                        : wn * (BNT / 2) + t * 32) + fr;

    const int64_t nk = static_cast<int64_t>(k_end - k_begin);  // K is a multiple of 64: nk >= 2
    mfma_stage::stage_loop<BNT, true>(lds, a_base, b_base, a_off, b_off, a_lds, b_lds, a_row, b_row, nk, acc);

    if constexpr (PARTIAL) {
        // Partial tile: the fp32 sums go to the workspace in accumulator order,
        // float4 (wave, mt, t, j, lane) holding elements 4j..4j+3 of n-tile t of
        // m-tile mt (partial_slot), so that each store writes 1 KiB contiguous.
        float* pt = partial + static_cast<int64_t>(unit) * TS::kPartialFloats;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    *reinterpret_cast<float4*>(pt + partial_slot<NT>(wave, mt, t, j, lane) * 4) =
                        make_float4(acc[mt][t][j * 4 + 0], acc[mt][t][j * 4 + 1], acc[mt][t][j * 4 + 2],
                                    acc[mt][t][j * 4 + 3]);
        return;
    }

    // Epilogue through LDS, so that global stores are whole rows: each wave
    // writes its bias-added bf16 outputs (GLU: silu(g) * u) into its own LDS
    // region, then reads it back row by row in 16-byte chunks and stores full
    // lines. Accumulator element v of lane l is row l % 32, column
    // 4 * (l / 32) + (v % 4) + 8 * (v / 4) of its 32x32 tile. Region rows are
    // kOutCols bf16; the 16-byte chunk c of row r sits at chunk c ^ (r & kSwz)
    // (conflict-free row reads). The GLU products of a 32x32 tile are formed
    // sixteen at a time, each step over all sixteen (independent exp and
    // reciprocal latencies overlap).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no stage copy may still be writing LDS
    bias_sh[tid] = bias_mine;
    __syncthreads();  // every wave is done reading the stages; the biases are in LDS
    constexpr int kOutCols = GLU ? BNT / 4 : BNT / 2;  // columns of a wave's output tile
    constexpr int kRowBytes = kOutCols * 2;
    constexpr int kChunks = kRowBytes / 16;   // 16-byte chunks per row
    constexpr int kSwz = kChunks - 1;
    static_assert(4 * 128 * kRowBytes <= kStages * kStageBytes, "output regions fit the stages");
    char* region = lds + wave * (128 * kRowBytes);
    const int col_base = GLU ? wn * (BNT / 4) : wn * (BNT / 2);  // within the block tile's columns
    constexpr int kOutTiles = GLU ? NT / 2 : NT;
#pragma unroll
    for (int nt = 0; nt < kOutTiles; ++nt) {
        // Biases of the 16 columns of n-tile nt (the same for every m-tile):
        // runs of four at col_base + nt * 32 + fg * 4 + 8 j (GLU value biases
        // BNT / 2 further on).
        float bias_g[16], bias_u[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int cl = col_base + nt * 32 + fg * 4 + j * 8;
            const float4 bg4 = *reinterpret_cast<const float4*>(&bias_sh[cl]);
            bias_g[j * 4 + 0] = bg4.x;
            bias_g[j * 4 + 1] = bg4.y;
            bias_g[j * 4 + 2] = bg4.z;
            bias_g[j * 4 + 3] = bg4.w;
            if constexpr (GLU) {
                const float4 bu4 = *reinterpret_cast<const float4*>(&bias_sh[BNT / 2 + cl]);
                bias_u[j * 4 + 0] = bu4.x;
                bias_u[j * 4 + 1] = bu4.y;
                bias_u[j * 4 + 2] = bu4.z;
                bias_u[j * 4 + 3] = bu4.w;
            }
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            // One 32x32 tile at a time: without the scheduling barrier every
            // accumulator is copied out of the AGPRs at once and VGPRs spill.
            __builtin_amdgcn_sched_barrier(0);
            const int r = mt * 32 + fr;
            float o[16];
            if constexpr (GLU) {
                float g[16], d[16];
#pragma unroll
                for (int v = 0; v < 16; ++v) g[v] = acc[mt][nt][v] + bias_g[v];
#pragma unroll
                for (int v = 0; v < 16; ++v) d[v] = __builtin_amdgcn_exp2f(g[v] * -1.4426950408889634f);
#pragma unroll
                for (int v = 0; v < 16; ++v) d[v] = __builtin_amdgcn_rcpf(1.0f + d[v]);
#pragma unroll
                for (int v = 0; v < 16; ++v) o[v] = (g[v] * d[v]) * (acc[mt][nt + NT / 2][v] + bias_u[v]);
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v) o[v] = acc[mt][nt][v] + bias_g[v];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int cl = nt * 32 + fg * 4 + j * 8;  // column within the wave tile
                union {
                    uint2 raw;
                    bf16 e[4];
                } w;
#pragma unroll
                for (int q = 0; q < 4; ++q) w.e[q] = from_f32<bf16>(o[j * 4 + q]);
                const int chunk = (cl >> 3) ^ (r & kSwz);
                *reinterpret_cast<uint2*>(region + r * kRowBytes + chunk * 16 + (cl & 4) * 2) = w.raw;
            }
        }
    }
    // Row-contiguous read-back (the wave's own region: LDS operations of a wave
    // complete in order) and full-line stores.
    // Eight reads are issued before their eight stores, so one LDS latency
    // covers eight lines.
    const int64_t out_col0 = n0 + col_base;
    constexpr int kIters = 128 * kChunks / kWave;
    constexpr int kBatch = 8;
    static_assert(kIters % kBatch == 0, "read-back batches");
#pragma unroll
    for (int b = 0; b < kIters; b += kBatch) {
        uint4 v[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int idx = (b + i) * kWave + lane;
            const int r = idx / kChunks, c = idx % kChunks;
            v[i] = *reinterpret_cast<const uint4*>(region + r * kRowBytes + ((c ^ (r & kSwz)) * 16));
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int idx = (b + i) * kWave + lane;
            const int r = idx / kChunks, c = idx % kChunks;
            const int64_t grow = row0 + wm * 128 + r;
            const int64_t col = out_col0 + c * 8;
            if (grow < row_end && col < n_out) *reinterpret_cast<uint4*>(C + grow * n_out + col) = v[i];
        }
    }
}

template <bool GLU, int BNT>
__global__ __launch_bounds__(kGemmThreads, TileShape<BNT>::kWgPerCu) void grouped_gemm_bf16_kernel(
    const bf16* __restrict__ A, const int64_t* __restrict__ a_index, int64_t a_count,
    const bf16* __restrict__ W0, const bf16* __restrict__ W1,
    const bf16* __restrict__ bias0, const bf16* __restrict__ bias1, bf16* __restrict__ C,
    const int32_t* __restrict__ slot_expert, const int64_t* __restrict__ slot_row,
    const int64_t* __restrict__ slot_end, int64_t n_out, int64_t K, int64_t max_slots, int64_t n_tiles,
    float* __restrict__ partial, uint32_t rounds) {
    using TS = TileShape<BNT>;
    constexpr int kStages = TS::kStages;
    constexpr uint32_t kStageBytes = TS::kStageBytes;
    __shared__ __attribute__((aligned(1024))) char lds[kStages * kStageBytes];
    __shared__ __attribute__((aligned(16))) float bias_sh[kGemmThreads];

    // One launch covers both kinds of workgroup. Whole tiles (blockIdx.x <
    // whole_grid, the most whole tiles the pairs can need, a multiple of 8):
    // the whole tiles of the split plan for the slots actually in use are
    // spread evenly over the eight XCDs (workgroup b runs on XCD b % 8) and the
    // surplus workgroups exit. Partial tiles (the kMaxSplitUnits workgroups
    // after them, dispatched as the last whole tiles run): workgroup
    // whole_grid + u takes unit u of the plan, K steps [k_begin, k_end) of its
    // leftover tile. `rounds` is the number of workgroups that run at once
    // (CUs x workgroups per CU).
    const uint32_t slots = static_cast<uint32_t>(min(static_cast<int64_t>(slot_expert[max_slots]), max_slots));
    const uint32_t nk_all = static_cast<uint32_t>(K / kBK);
    const SplitPlan plan = split_plan(slots * static_cast<uint32_t>(n_tiles), nk_all, rounds);
    const uint32_t whole_grid = static_cast<uint32_t>((max_slots * n_tiles + 7) / 8 * 8);
    const bool partial_unit = blockIdx.x >= whole_grid;
    if (!partial_unit) {
        const uint32_t per_xcd = (plan.whole + 7) / 8;
        if ((blockIdx.x >> 3) >= per_xcd) return;
        const uint32_t logical = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
        if (logical >= plan.whole) return;
        gemm_tile<GLU, false, BNT>(A, a_index, a_count, W0, W1, bias0, bias1, C, slot_expert, slot_row, slot_end,
                                   n_out, K, n_tiles, partial, lds, bias_sh, logical, slots, 0, 0, nk_all);
    } else {
        const uint32_t unit = blockIdx.x - whole_grid;
        if (unit >= plan.units) return;
        const uint32_t logical = plan.whole + unit / plan.split;
        const uint32_t chunk = unit % plan.split;
        gemm_tile<GLU, true, BNT>(A, a_index, a_count, W0, W1, bias0, bias1, C, slot_expert, slot_row, slot_end,
                                  n_out, K, n_tiles, partial, lds, bias_sh, logical, slots, unit,
                                  chunk * nk_all / plan.split, (chunk + 1) * nk_all / plan.split);
    }
}

// Sums the partial tiles of the split plan in chunk order, adds the biases
// (GLU: silu(g + b_g) * (u + b_v)) and writes the bf16 outputs. A thread takes
// one float4 slot of a leftover tile (GLU: a gate slot, n-tile t < 2, and its
// value slot t + 2), reading the slot in every chunk (coalesced), and writes
// the four consecutive outputs it holds: row wm * 128 + mt * 32 + lane % 32,
// columns col_base + t * 32 + 4 (lane / 32) + 8 j (+0..3).
template <bool GLU, int BNT>
__global__ __launch_bounds__(256) void split_fixup_kernel(
    const float* __restrict__ partial, const bf16* __restrict__ bias0, const bf16* __restrict__ bias1,
    bf16* __restrict__ C, const int32_t* __restrict__ slot_expert, const int64_t* __restrict__ slot_row,
    const int64_t* __restrict__ slot_end, int64_t n_out, int64_t K, int64_t max_slots, int64_t n_tiles,
    uint32_t rounds) {
    using TS = TileShape<BNT>;
    constexpr int NT = TS::kNT;
    constexpr int64_t kTileFloats = TS::kPartialFloats;
    const uint32_t slots = static_cast<uint32_t>(min(static_cast<int64_t>(slot_expert[max_slots]), max_slots));
    const SplitPlan plan = split_plan(slots * static_cast<uint32_t>(n_tiles), static_cast<uint32_t>(K / kBK), rounds);
    if (plan.units == 0) return;
    constexpr uint32_t kSlotsPerTile = GLU ? kTileFloats / 8 : kTileFloats / 4;
    const uint32_t items = plan.units / plan.split * kSlotsPerTile;
    for (uint32_t item = blockIdx.x * blockDim.x + threadIdx.x; item < items; item += gridDim.x * blockDim.x) {
        const uint32_t rt = item / kSlotsPerTile;
        uint32_t f = item % kSlotsPerTile;
        const int lane = static_cast<int>(f % kWave);
        f /= kWave;
        const int j = static_cast<int>(f % 4);
        f /= 4;
        const int t = static_cast<int>(f % (GLU ? NT / 2 : NT));
        f /= GLU ? NT / 2 : NT;
        const int mt = static_cast<int>(f % 4);
        const int wave = static_cast<int>(f / 4);
        const int wm = wave >> 1, wn = wave & 1;
        uint32_t slot, tile_n;
        tile_coords(plan.whole + rt, slots, static_cast<uint32_t>(n_tiles), slot, tile_n);
        const int e = slot_expert[slot];
        const int64_t grow = slot_row[slot] + wm * 128 + mt * 32 + (lane & 31);
        if (e < 0 || grow >= slot_end[slot]) continue;
        const float* pt = partial + static_cast<int64_t>(rt) * plan.split * kTileFloats;
        const int64_t s0 = partial_slot<NT>(wave, mt, t, j, lane) * 4;
        // Chunks are loaded eight at a time and added in chunk order; chunks
        // past the split read as +0, which leaves a sum that starts at +0
        // unchanged.
        const int64_t sv = partial_slot<NT>(wave, mt, GLU ? t + NT / 2 : t, j, lane) * 4;
        float4 g = make_float4(0.0f, 0.0f, 0.0f, 0.0f), u = g;
        for (uint32_t k0 = 0; k0 < plan.split; k0 += 8) {
            float4 pg[8], pu[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const bool in = k0 + i < plan.split;
                const int64_t base = static_cast<int64_t>(in ? k0 + i : 0) * kTileFloats;
                pg[i] = *reinterpret_cast<const float4*>(pt + base + s0);
                if (!in) pg[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if constexpr (GLU) {
                    pu[i] = *reinterpret_cast<const float4*>(pt + base + sv);
                    if (!in) pu[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                g.x += pg[i].x;
                g.y += pg[i].y;
                g.z += pg[i].z;
                g.w += pg[i].w;
                if constexpr (GLU) {
                    u.x += pu[i].x;
                    u.y += pu[i].y;
                    u.z += pu[i].z;
                    u.w += pu[i].w;
                }
            }
        }
        const int64_t col = (GLU ? static_cast<int64_t>(tile_n) * (BNT / 2) + wn * (BNT / 4)
                                 : static_cast<int64_t>(tile_n) * BNT + wn * (BNT / 2)) +
                            t * 32 + (lane >> 5) * 4 + j * 8;
        if (col >= n_out) continue;
        const int64_t bo = static_cast<int64_t>(e) * n_out + col;
        const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
        union {
            uint2 raw;
            bf16 h[4];
        } w;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if constexpr (GLU) w.h[c] = from_f32<bf16>(silu_f(gv[c] + to_f32(bias0[bo + c])) * (uv[c] + to_f32(bias1[bo + c])));
            else w.h[c] = from_f32<bf16>(gv[c] + to_f32(bias0[bo + c]));
        }
        *reinterpret_cast<uint2*>(C + grow * n_out + col) = w.raw;
    }
}

// ------------------------------------------------- fp32-accumulating SIMT path
// One 256-thread block per sorted pair (the reference's decomposition), used for
// float32 / float16 weights and for shapes the MFMA tiles do not cover.
template <typename T>
__global__ __launch_bounds__(256) void glu_hidden_simt_kernel(
    const T* __restrict__ x, const int64_t* __restrict__ experts, const int64_t* __restrict__ offsets, int64_t E,
    const T* __restrict__ Wg, const T* __restrict__ bg, const T* __restrict__ Wv, const T* __restrict__ bv,
    float* __restrict__ H, int64_t D, int64_t Hd) {
    const int64_t p = blockIdx.x;
    if (p >= offsets[E]) return;  // the grid covers exactly the pairs, so p < pairs
    const int64_t e = experts[p];
    if (e < 0 || e >= E) return;
    const T* xr = x + p * D;
    for (int64_t h = threadIdx.x; h < Hd; h += 256) {
        const T* wg = Wg + (e * Hd + h) * D;
        const T* wv = Wv + (e * Hd + h) * D;
        float g = to_f32(bg[e * Hd + h]), u = to_f32(bv[e * Hd + h]);
        for (int64_t c = 0; c < D; ++c) {
            const float xv = to_f32(xr[c]);
            g = __builtin_fmaf(xv, to_f32(wg[c]), g);
            u = __builtin_fmaf(xv, to_f32(wv[c]), u);
        }
        H[p * Hd + h] = silu_f(g) * u;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void glu_output_simt_kernel(
    const float* __restrict__ H, const int64_t* __restrict__ experts, const int64_t* __restrict__ offsets, int64_t E,
    const T* __restrict__ Wo, const T* __restrict__ bo, T* __restrict__ y, int64_t D, int64_t Hd) {
    const int64_t p = blockIdx.x;
    if (p >= offsets[E]) return;
    const int64_t e = experts[p];
    if (e < 0 || e >= E) return;
    const float* hr = H + p * Hd;
    for (int64_t c = threadIdx.x; c < D; c += 256) {
        const T* wo = Wo + (e * D + c) * Hd;
        float acc = to_f32(bo[e * D + c]);
        for (int64_t h = 0; h < Hd; ++h) acc = __builtin_fmaf(hr[h], to_f32(wo[h]), acc);
        y[p * D + c] = from_f32<T>(acc);
    }
}

// ------------------------------------------------------------ skinny path ---
// Few rows per expert (a decode step: 64 tokens x top-2 over 16 experts is
// about 8 rows each). The big tiles above would run 256-row MFMA tiles for 8
// useful rows, so the step would be bound by wasted matrix work; here it is
// bound by streaming the expert weights once. A task is 32 output columns of
// one expert (GLU: 32 hidden units, their gate and value rows) over every row
// of that expert, in passes of 32 rows (one MFMA block). S waves share a task
// by K, in interleaved 64-wide steps (adjacent 128-byte pieces of each weight
// row), and add their partial sums through LDS; with S = 1 a wave owns its
// task alone, G tasks per workgroup, with no LDS and no barrier, and the
// epilogue reads its accumulators directly. Each wave keeps PF steps of loads
// in flight (a ring of PF register sets). Operands come straight from global
// memory in the MFMA register layout: lane l holds row l % 32 and, per step,
// the 32 contiguous values of half l / 32, of which MFMA j takes values
// 8j..8j+7; A and B use the same assignment, so every product pairs equal k.
// Rows past the segment are not loaded (zero fragments) and not stored.
//
// FRAG: the weights are in fragment order (koemi_moe_weights_to_fragments):
// each 32-row block of a weight matrix is stored as [K / 64 steps][4 loads]
// [64 lanes][8 values], so that every load instruction of a wave reads 1 KB
// of contiguous memory and a task streams its 32 x K block front to back
// (with row-major weights each load touches 32 rows, 32 bytes apiece). The
// same products in the same order: results equal the row-major path's bit for
// bit.
constexpr int kSkinnyCols = 32;
constexpr int64_t kSkinnyMaxRowsPerExpert = 64;  // average over experts below which the path is used
#ifndef KOEMI_SKINNY_GLU
#define KOEMI_SKINNY_GLU 2, 1, 2  // S, G, PF of the GLU (first) GEMM
#endif
#ifndef KOEMI_SKINNY_OUT
#define KOEMI_SKINNY_OUT 4, 1, 2  // S, G, PF of the output GEMM
#endif

template <bool GLU, bool FRAG, int S, int G, int PF>
__global__ __launch_bounds__(S * G * kWave) void skinny_gemm_kernel(
    const bf16* __restrict__ a, const int64_t* __restrict__ a_index, int64_t a_count,
    const bf16* __restrict__ w0, const bf16* __restrict__ w1,
    const bf16* __restrict__ bias0, const bf16* __restrict__ bias1, bf16* __restrict__ c,
    const int64_t* __restrict__ offsets, int64_t n_out, int64_t K, int64_t col_groups, int64_t experts,
    int64_t pairs) {
    static_assert(S == 1 || G == 1, "waves that split K share one task per workgroup (the barriers)");
    constexpr int kMats = GLU ? 2 : 1;
    __shared__ float red[S > 1 ? S : 1][kMats][S > 1 ? 16 : 1][kWave];
    const int64_t task_blocks = (experts * col_groups + G - 1) / G;
    if (static_cast<int64_t>(blockIdx.x) >= task_blocks) {
        // workgroups past the tasks zero the rows past the valid pairs
        // (moe_kernels.cu:512, 167-169), a grid stride over those rows
        const int64_t extra = gridDim.x - task_blocks;
        const int64_t start = min(max(offsets[experts], int64_t(0)), pairs);
        for (int64_t p = start + (blockIdx.x - task_blocks); p < pairs; p += extra)
            for (int64_t q = threadIdx.x; q < n_out; q += blockDim.x) c[p * n_out + q] = from_f32<bf16>(0.0f);
        return;
    }
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int split = wave % S;
    const int64_t task = static_cast<int64_t>(blockIdx.x) * G + wave / S;
    if (task >= experts * col_groups) return;  // S == 1 here (G > 1): no barrier follows
    const int64_t e = task / col_groups;
    const int64_t n0 = (task % col_groups) * kSkinnyCols;
    const int64_t row0 = offsets[e];
    const int64_t count = offsets[e + 1] - row0;
    if (count <= 0) return;  // uniform over the task's waves
    const int r = lane % 32, half = lane / 32;
    const int64_t steps = K / 64;
    // this lane's first weight value: row r, values [32 half, + 32) of each
    // step; in fragment order the lane's 16 bytes of load j of step k start
    // at (4 k + j) 512 + 8 lane within the 32-row block
    const int64_t w_lane = FRAG ? 8 * lane : r * K + 32 * half;
    const bf16* wr0 = w0 + (e * n_out + n0) * K + w_lane;
    const bf16* wr1 = GLU ? w1 + (e * n_out + n0) * K + w_lane : wr0;
    const int64_t col = n0 + r;
    const float b0 = to_f32(bias0[e * n_out + col]);
    const float b1 = GLU ? to_f32(bias1[e * n_out + col]) : 0.0f;
    struct Frags {
        bf16x8 w[kMats][4];
        bf16x8 x[4];
    };
    for (int64_t pass = 0; pass < count; pass += 32) {
        const int64_t rows = count - pass < 32 ? count - pass : 32;
        const bool aok = r < rows;
        int64_t arow = row0 + pass + (aok ? r : 0);
        if (a_index) arow = min(max(a_index[arow], int64_t(0)), a_count - 1);  // a row of the unsorted context
        const bf16* ar = a + arow * K + 32 * half;
        f32x16 acc[kMats];
#pragma unroll
        for (int m = 0; m < kMats; ++m)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[m][i] = 0.0f;
        auto load = [&](int64_t step, Frags& f) {
            if (step >= steps) return;
            const int64_t k = step * 64;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t at = FRAG ? (step * 4 + j) * 512 : k + 8 * j;
                f.w[0][j] = *reinterpret_cast<const bf16x8*>(wr0 + at);
                if constexpr (GLU) f.w[1][j] = *reinterpret_cast<const bf16x8*>(wr1 + at);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                bf16x8 v = {};
                if (aok) v = *reinterpret_cast<const bf16x8*>(ar + k + 8 * j);
                f.x[j] = v;
            }
        };
        auto multiply = [&](int64_t step, const Frags& f) {
            if (step >= steps) return;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int m = 0; m < kMats; ++m)
                    acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.x[j], f.w[m][j], acc[m], 0, 0, 0);
        };
        // this wave's steps are split, split + S, ...; set p of the ring holds
        // the step p (mod PF) of them, loaded PF steps before its multiply
        Frags f[PF];
#pragma unroll
        for (int p = 0; p < PF; ++p) load(split + p * S, f[p]);
        for (int64_t s0 = split; s0 < steps; s0 += PF * S) {
#pragma unroll
            for (int p = 0; p < PF; ++p) {
                multiply(s0 + p * S, f[p]);
                load(s0 + (p + PF) * S, f[p]);
            }
        }
        // entry i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32
        if constexpr (S == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t row = 8 * (i / 4) + 4 * half + i % 4;
                if (row >= rows) continue;
                float out;
                if constexpr (GLU) out = silu_f(acc[0][i] + b0) * (acc[kMats - 1][i] + b1);
                else out = acc[0][i] + b0;
                c[(row0 + pass + row) * n_out + col] = from_f32<bf16>(out);
            }
        } else {
#pragma unroll
            for (int m = 0; m < kMats; ++m)
#pragma unroll
                for (int i = 0; i < 16; ++i) red[split][m][i][lane] = acc[m][i];
            __syncthreads();
            // 16 accumulator entries x 64 lanes = 1024 outputs, 16 / S per thread
#pragma unroll
            for (int q = 0; q < 16 / S; ++q) {
                const int i = q * S + split;  // wave-uniform
                const int64_t row = 8 * (i / 4) + 4 * half + i % 4;
                if (row >= rows) continue;
                float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
                for (int w = 0; w < S; ++w) {
                    v0 += red[w][0][i][lane];
                    if constexpr (GLU) v1 += red[w][kMats - 1][i][lane];
                }
                float out;
                if constexpr (GLU) out = silu_f(v0 + b0) * (v1 + b1);
                else out = v0 + b0;
                c[(row0 + pass + row) * n_out + col] = from_f32<bf16>(out);
            }
            __syncthreads();  // red is rewritten by the next pass
        }
    }
}

// Launch of skinny_gemm_kernel<GLU, FRAG, S, G, PF> over every task (plus
// `tail_wgs` workgroups that zero the rows past the valid pairs).
template <bool GLU, bool FRAG, int S, int G, int PF>
void launch_skinny(const bf16* a, const int64_t* a_index, int64_t a_count, const bf16* w0, const bf16* w1,
                   const bf16* bias0, const bf16* bias1, bf16* c, const int64_t* offsets, int64_t n_out, int64_t K,
                   int64_t experts, int64_t pairs, int64_t tail_wgs, hipStream_t s) {
    const int64_t groups = n_out / kSkinnyCols;
    const int64_t blocks = (experts * groups + G - 1) / G + tail_wgs;
    hipLaunchKernelGGL((skinny_gemm_kernel<GLU, FRAG, S, G, PF>), dim3(static_cast<unsigned>(blocks)), dim3(S * G * kWave),
                       0, s, a, a_index, a_count, w0, w1, bias0, bias1, c, offsets, n_out, K, groups, experts, pairs);
}

// Both GEMMs of the skinny path: GEMM 1 into the bf16 hidden rows H, GEMM 2
// into y (with zero_tail, extra workgroups of its launch zero the rows past
// the valid pairs).
template <bool FRAG>
int run_skinny(const void* x, const int64_t* x_index, int64_t x_rows, const int64_t* offsets, const void* Wg,
               const void* bg, const void* Wv, const void* bv, const void* Wo, const void* bo, void* y, int64_t P,
               int64_t D, int64_t Hd, int64_t E, bf16* H, hipStream_t s, bool zero_tail) {
    launch_skinny<true, FRAG, KOEMI_SKINNY_GLU>(static_cast<const bf16*>(x), x_index, x_rows, static_cast<const bf16*>(Wg),
                                                static_cast<const bf16*>(Wv), static_cast<const bf16*>(bg),
                                                static_cast<const bf16*>(bv), H, offsets, Hd, D, E, P, 0, s);
    int st = check_launch("koemi_moe_grouped_mlp(skinny gemm1)");
    if (st != KOEMI_OK) return st;
    const int64_t tail_wgs = zero_tail ? (P < 64 ? P : 64) : 0;
    launch_skinny<false, FRAG, KOEMI_SKINNY_OUT>(H, nullptr, P, static_cast<const bf16*>(Wo),
                                                 static_cast<const bf16*>(Wo), static_cast<const bf16*>(bo),
                                                 static_cast<const bf16*>(bo), static_cast<bf16*>(y), offsets, D, Hd, E,
                                                 P, tail_wgs, s);
    return check_launch("koemi_moe_grouped_mlp(skinny gemm2)");
}

// Weights [matrices, rows, cols] bf16 into fragment order: thread t writes
// the 16 bytes of chunk t of the destination, which in its 32-row block is
// lane l = t % 64 of load j = (t / 64) % 4 of step k = t / 256: row l % 32 of
// the block, columns 64 k + 32 (l / 32) + 8 j .. + 8.
__global__ void weights_to_fragments_kernel(const bf16x8* __restrict__ src, bf16x8* __restrict__ dst,
                                            int64_t chunks, int64_t cols) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= chunks) return;
    const int64_t block_chunks = 4 * cols;  // 32 rows x cols values / 8
    const int64_t block = t / block_chunks, c = t % block_chunks;
    const int64_t lane = c % 64, j = (c / 64) % 4, step = c / 256;
    const int64_t row = block * 32 + lane % 32;
    const int64_t col = step * 64 + 32 * (lane / 32) + 8 * j;
    dst[t] = src[(row * cols + col) / 8];
}

// Rows past the valid pairs are zero (moe_kernels.cu:512, 167-169); a
// grid-stride loop over only those rows.
template <typename T>
__global__ void zero_tail_rows_kernel(T* __restrict__ y, const int64_t* __restrict__ valid_end, int64_t pairs,
                                      int64_t D) {
    const int64_t start = min(max(*valid_end, int64_t(0)), pairs);
    for (int64_t p = start + blockIdx.x; p < pairs; p += gridDim.x)
        for (int64_t c = threadIdx.x; c < D; c += blockDim.x) y[p * D + c] = static_cast<T>(0.0f);
}

inline unsigned tail_blocks(int64_t pairs) { return static_cast<unsigned>(pairs < 1024 ? (pairs > 0 ? pairs : 1) : 1024); }

template <typename T>
int run_simt(const void* x, const int64_t* experts, const int64_t* offsets, const void* Wg, const void* bg,
             const void* Wv, const void* bv, const void* Wo, const void* bo, void* y, int64_t P, int64_t D, int64_t Hd,
             int64_t E, float* H, hipStream_t s) {
    if (P > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many pairs for the SIMT grouped MLP");
    const dim3 grid(static_cast<unsigned>(P)), block(256);
    hipLaunchKernelGGL(glu_hidden_simt_kernel<T>, grid, block, 0, s, static_cast<const T*>(x), experts, offsets, E,
                       static_cast<const T*>(Wg), static_cast<const T*>(bg), static_cast<const T*>(Wv),
                       static_cast<const T*>(bv), H, D, Hd);
    int st = check_launch("koemi_moe_grouped_mlp(hidden)");
    if (st != KOEMI_OK) return st;
    hipLaunchKernelGGL(glu_output_simt_kernel<T>, grid, block, 0, s, H, experts, offsets, E, static_cast<const T*>(Wo),
                       static_cast<const T*>(bo), static_cast<T*>(y), D, Hd);
    st = check_launch("koemi_moe_grouped_mlp(output)");
    if (st != KOEMI_OK) return st;
    hipLaunchKernelGGL(zero_tail_rows_kernel<T>, dim3(tail_blocks(P)), block, 0, s, static_cast<T*>(y), offsets + E, P, D);
    return check_launch("koemi_moe_grouped_mlp(zero)");
}

// Compute units of the current device (the rounds of one-workgroup-per-CU tiles).
int64_t device_cus() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] > 0) return cached[dev];
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    cached[dev] = n;
    return n;
}

// x_index (or null): GEMM 1 reads context row x_index[i] (of x_rows) for pair i.
// zero_tail: the rows past the valid pairs are zeroed (the reference's output
// contract); the indexed entry leaves them, as nothing reads them.
int run_mfma(const void* x, const int64_t* x_index, int64_t x_rows, const int64_t* offsets, const void* Wg,
             const void* bg, const void* Wv, const void* bv, const void* Wo, const void* bo, void* y, int64_t P,
             int64_t D, int64_t Hd, int64_t E, const MlpWorkspace& ws, char* base, hipStream_t s, bool zero_tail) {
    bf16* H = reinterpret_cast<bf16*>(base + ws.hidden_off);
    int32_t* slot_expert = reinterpret_cast<int32_t*>(base + ws.slot_expert_off);
    int64_t* slot_row = reinterpret_cast<int64_t*>(base + ws.slot_row_off);
    int64_t* slot_end = reinterpret_cast<int64_t*>(base + ws.slot_end_off);
    float* partial = reinterpret_cast<float*>(base + ws.partial_off);
    if (ws.max_slots > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many tiles");
    if (Hd * D > 0x7fffffffLL || 256 * (Hd > D ? Hd : D) > 0x7fffffffLL)  // 32-bit byte offsets in the tiles
        return fail(KOEMI_ERR_UNSUPPORTED, "grouped MLP needs hidden * width < 2^31");
    if (E > kMaxScheduleExperts) return fail(KOEMI_ERR_UNSUPPORTED, "grouped MLP supports at most %lld experts",
                                             static_cast<long long>(kMaxScheduleExperts));
    if (P <= kSkinnyMaxRowsPerExpert * E && E * ((Hd > D ? Hd : D) / kSkinnyCols) <= 0x7fffffffLL) {
        return run_skinny<false>(x, x_index, x_rows, offsets, Wg, bg, Wv, bv, Wo, bo, y, P, D, Hd, E, H, s, zero_tail);
    }
    hipLaunchKernelGGL(build_schedule_kernel, dim3(1), dim3(kSchedThreads), static_cast<size_t>(E + 1) * sizeof(int32_t),
                       s, offsets, E, P, ws.max_slots, slot_expert, slot_row, slot_end);
    int st = check_launch("koemi_moe_grouped_mlp(schedule)");
    if (st != KOEMI_OK) return st;
    const int64_t slots = ws.max_slots;
    constexpr int BNT = KOEMI_GEMM_BN;
    const uint32_t rounds = static_cast<uint32_t>(device_cus() * TileShape<BNT>::kWgPerCu);
    // Whole tiles, then the partial tiles of the split plan (if any; every
    // workgroup exits otherwise), then their sums.
    auto launch = [&](auto kernel, auto fixup, const bf16* a, const int64_t* a_index,
                      int64_t a_count, const void* w0, const void* w1, const void* b0, const void* b1, bf16* c,
                      int64_t n_out, int64_t K, int64_t n_tiles, const char* what) {
        // whole tiles, then the partial units, in one launch
        const int64_t whole_grid = (slots * n_tiles + 7) / 8 * 8;
        if (whole_grid + kMaxSplitUnits > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many tiles");
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(whole_grid + kMaxSplitUnits)), dim3(kGemmThreads), 0, s,
                           a, a_index, a_count, static_cast<const bf16*>(w0), static_cast<const bf16*>(w1),
                           static_cast<const bf16*>(b0), static_cast<const bf16*>(b1), c, slot_expert, slot_row,
                           slot_end, n_out, K, slots, n_tiles, partial, rounds);
        int st2 = check_launch(what);
        if (st2 != KOEMI_OK) return st2;
        // At most kMaxSplitUnits / 2 leftover tiles of 8192 (GLU) or 16384 slots.
        hipLaunchKernelGGL(fixup, dim3(1024), dim3(256), 0, s, partial, static_cast<const bf16*>(b0),
                           static_cast<const bf16*>(b1), c, slot_expert, slot_row, slot_end, n_out, K, slots,
                           n_tiles, rounds);
        return check_launch(what);
    };
    st = launch(grouped_gemm_bf16_kernel<true, BNT>, split_fixup_kernel<true, BNT>, static_cast<const bf16*>(x), x_index, x_rows, Wg, Wv, bg, bv, H, Hd, D,
                (Hd + BNT / 2 - 1) / (BNT / 2), "koemi_moe_grouped_mlp(gemm1)");
    if (st != KOEMI_OK) return st;
    st = launch(grouped_gemm_bf16_kernel<false, BNT>, split_fixup_kernel<false, BNT>, H, static_cast<const int64_t*>(nullptr), P, Wo, Wo, bo, bo,
                static_cast<bf16*>(y), D, Hd, (D + BNT - 1) / BNT,
                "koemi_moe_grouped_mlp(gemm2)");
    if (st != KOEMI_OK) return st;
    if (!zero_tail) return KOEMI_OK;
    hipLaunchKernelGGL(zero_tail_rows_kernel<bf16>, dim3(tail_blocks(P)), dim3(256), 0, s, static_cast<bf16*>(y),
                       offsets + E, P, D);
    return check_launch("koemi_moe_grouped_mlp(zero)");
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" size_t koemi_moe_grouped_mlp_workspace_bytes(int64_t pairs, int64_t width, int64_t hidden,
                                                        int64_t expert_count, int dtype) {
    if (pairs < 0 || width < 1 || hidden < 1 || expert_count < 1) return 0;
    return mlp_workspace(pairs, width, hidden, expert_count, dtype).total;
}

extern "C" int koemi_moe_grouped_mlp(const void* sorted_context, const int64_t* sorted_experts,
                                     const int64_t* segment_offsets, const void* gate_weights,
                                     const void* gate_biases, const void* value_weights, const void* value_biases,
                                     const void* output_weights, const void* output_biases, void* output,
                                     int64_t pairs, int64_t width, int64_t hidden, int64_t expert_count, int dtype,
                                     void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (pairs < 0 || width < 1 || hidden < 1 || expert_count < 1)
        return fail(KOEMI_ERR_INVALID, "grouped MLP needs positive width, hidden and expert_count");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "grouped MLP does not support dtype %s", dtype_name(dtype));
    if (pairs == 0) return KOEMI_OK;
    if (!sorted_context || !sorted_experts || !segment_offsets || !gate_weights || !gate_biases || !value_weights ||
        !value_biases || !output_weights || !output_biases || !output)
        return fail(KOEMI_ERR_INVALID, "grouped MLP received a null pointer");
    const MlpWorkspace ws = mlp_workspace(pairs, width, hidden, expert_count, dtype);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "grouped MLP workspace too small: need %zu bytes", ws.total);
    char* base = static_cast<char*>(workspace);
    hipStream_t s = as_stream(stream);
    const bool aligned = reinterpret_cast<uintptr_t>(sorted_context) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(gate_weights) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(value_weights) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(output_weights) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(output) % 16 == 0;
    if (mfma_shape(width, hidden, dtype) && !aligned)
        return fail(KOEMI_ERR_INVALID, "grouped MLP bf16 operands must be 16-byte aligned");
    if (mfma_shape(width, hidden, dtype))
        return run_mfma(sorted_context, nullptr, pairs, segment_offsets, gate_weights, gate_biases, value_weights,
                        value_biases, output_weights, output_biases, output, pairs, width, hidden, expert_count, ws,
                        base, s, true);
    float* H = reinterpret_cast<float*>(base + ws.hidden_off);
    switch (dtype) {
        case KOEMI_F32:
            return run_simt<float>(sorted_context, sorted_experts, segment_offsets, gate_weights, gate_biases,
                                   value_weights, value_biases, output_weights, output_biases, output, pairs, width,
                                   hidden, expert_count, H, s);
        case KOEMI_F16:
            return run_simt<f16>(sorted_context, sorted_experts, segment_offsets, gate_weights, gate_biases,
                                 value_weights, value_biases, output_weights, output_biases, output, pairs, width,
                                 hidden, expert_count, H, s);
        default:
            return run_simt<bf16>(sorted_context, sorted_experts, segment_offsets, gate_weights, gate_biases,
                                  value_weights, value_biases, output_weights, output_biases, output, pairs, width,
                                  hidden, expert_count, H, s);
    }
}

extern "C" int koemi_moe_grouped_mlp_indexed(const void* context, int64_t tokens, const int64_t* sorted_rows,
                                             const int64_t* segment_offsets, const void* gate_weights,
                                             const void* gate_biases, const void* value_weights,
                                             const void* value_biases, const void* output_weights,
                                             const void* output_biases, void* output, int64_t pairs, int64_t width,
                                             int64_t hidden, int64_t expert_count, void* workspace,
                                             size_t workspace_bytes, koemi_stream_t stream) {
    if (pairs < 0 || tokens < 1 || width < 1 || hidden < 1 || expert_count < 1)
        return fail(KOEMI_ERR_INVALID, "grouped MLP needs positive tokens, width, hidden and expert_count");
    if (!mfma_shape(width, hidden, KOEMI_BF16))
        return fail(KOEMI_ERR_UNSUPPORTED, "the indexed grouped MLP needs width and hidden multiples of %d", kKAlign);
    if (pairs == 0) return KOEMI_OK;
    if (!context || !sorted_rows || !segment_offsets || !gate_weights || !gate_biases || !value_weights ||
        !value_biases || !output_weights || !output_biases || !output)
        return fail(KOEMI_ERR_INVALID, "grouped MLP received a null pointer");
    if (tokens * width > 0x7fffffffLL)  // 32-bit byte offsets of context rows
        return fail(KOEMI_ERR_UNSUPPORTED, "the indexed grouped MLP needs tokens * width < 2^31");
    const MlpWorkspace ws = mlp_workspace(pairs, width, hidden, expert_count, KOEMI_BF16);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "grouped MLP workspace too small: need %zu bytes", ws.total);
    const bool aligned = reinterpret_cast<uintptr_t>(context) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(gate_weights) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(value_weights) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(output_weights) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(output) % 16 == 0;
    if (!aligned) return fail(KOEMI_ERR_INVALID, "grouped MLP bf16 operands must be 16-byte aligned");
    return run_mfma(context, sorted_rows, tokens, segment_offsets, gate_weights, gate_biases, value_weights,
                    value_biases, output_weights, output_biases, output, pairs, width, hidden, expert_count, ws,
                    static_cast<char*>(workspace), as_stream(stream), false);
}

extern "C" int koemi_moe_weights_to_fragments(const void* weights, void* fragments, int64_t matrices, int64_t rows,
                                              int64_t cols, koemi_stream_t stream) {
    if (matrices < 1 || rows < 1 || cols < 1 || rows % 32 != 0 || cols % 64 != 0)
        return fail(KOEMI_ERR_INVALID, "fragment order needs rows a multiple of 32 and cols a multiple of 64");
    if (!weights || !fragments) return fail(KOEMI_ERR_INVALID, "fragment order received a null pointer");
    if (reinterpret_cast<uintptr_t>(weights) % 16 != 0 || reinterpret_cast<uintptr_t>(fragments) % 16 != 0)
        return fail(KOEMI_ERR_INVALID, "fragment order needs 16-byte aligned weights");
    if (weights == fragments) return fail(KOEMI_ERR_INVALID, "fragment order cannot run in place");
    const int64_t chunks = matrices * rows * cols / 8;
    if (chunks / 256 + 1 > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many weights to reorder");
    hipLaunchKernelGGL(weights_to_fragments_kernel, dim3(static_cast<unsigned>((chunks + 255) / 256)), dim3(256), 0,
                       as_stream(stream), static_cast<const bf16x8*>(weights), static_cast<bf16x8*>(fragments), chunks,
                       cols);
    return check_launch("koemi_moe_weights_to_fragments");
}

extern "C" int koemi_moe_grouped_mlp_fragments(const void* context, int64_t tokens, const int64_t* sorted_rows,
                                               const int64_t* segment_offsets, const void* gate_fragments,
                                               const void* gate_biases, const void* value_fragments,
                                               const void* value_biases, const void* output_fragments,
                                               const void* output_biases, void* output, int64_t pairs, int64_t width,
                                               int64_t hidden, int64_t expert_count, void* workspace,
                                               size_t workspace_bytes, koemi_stream_t stream) {
    if (pairs < 0 || tokens < 1 || width < 1 || hidden < 1 || expert_count < 1)
        return fail(KOEMI_ERR_INVALID, "grouped MLP needs positive tokens, width, hidden and expert_count");
    if (!mfma_shape(width, hidden, KOEMI_BF16))
        return fail(KOEMI_ERR_UNSUPPORTED, "the fragment-order grouped MLP needs width and hidden multiples of %d",
                    kKAlign);
    if (pairs > kSkinnyMaxRowsPerExpert * expert_count)
        return fail(KOEMI_ERR_UNSUPPORTED, "the fragment-order grouped MLP takes at most %lld pairs per expert on "
                    "average (the few-rows path)", static_cast<long long>(kSkinnyMaxRowsPerExpert));
    if (pairs == 0) return KOEMI_OK;
    if (!context || !sorted_rows || !segment_offsets || !gate_fragments || !gate_biases || !value_fragments ||
        !value_biases || !output_fragments || !output_biases || !output)
        return fail(KOEMI_ERR_INVALID, "grouped MLP received a null pointer");
    if (tokens * width > 0x7fffffffLL)
        return fail(KOEMI_ERR_UNSUPPORTED, "the indexed grouped MLP needs tokens * width < 2^31");
    const MlpWorkspace ws = mlp_workspace(pairs, width, hidden, expert_count, KOEMI_BF16);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "grouped MLP workspace too small: need %zu bytes", ws.total);
    const bool aligned = reinterpret_cast<uintptr_t>(context) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(gate_fragments) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(value_fragments) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(output_fragments) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(output) % 16 == 0;
    if (!aligned) return fail(KOEMI_ERR_INVALID, "grouped MLP bf16 operands must be 16-byte aligned");
    bf16* H = reinterpret_cast<bf16*>(static_cast<char*>(workspace) + ws.hidden_off);
    return run_skinny<true>(context, sorted_rows, tokens, segment_offsets, gate_fragments, gate_biases, value_fragments,
                            value_biases, output_fragments, output_biases, output, pairs, width, hidden, expert_count,
                            H, as_stream(stream), false);
}
