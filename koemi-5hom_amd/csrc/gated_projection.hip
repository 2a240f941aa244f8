// Gate projection and working-state scan of a HERM window in one kernel.
//
// Reference: model/memory.py:14-30 (BoundedRecurrentState.gates: the two
// width x width projections W_r u + b_r, W_c u + b_c, the sigmoid retention
// and the tanh candidate) with the masking of network.py:307-309 and the scan
// h_t = a_t h_{t-1} + b_t of network.py:310, under bf16 autocast (the
// projection's results are bf16, its bias added in fp32 before the rounding).
// The reference computes the projections as two GEMMs whose outputs go
// through HBM, then the gates and the scan as torch operations.
//
// Here the stacked weight [W_r ; W_c] (bf16, [2F, K]) is multiplied on bf16
// MFMA (the main loop of mfma_stage.hpp) in block tiles of 256 consecutive
// positions of one sequence x 64 (or 128) features: the B tile holds the
// retention rows and the candidate rows of the same features, so a lane's
// accumulators hold, for one feature, the retention and candidate
// pre-activations of sixteen positions, and the epilogue forms the gates and
// scans them without the pre-activations leaving the registers:
//
//   1. a, b of every position in place of the accumulators (the pre-activation
//      rounded to bf16 after the bias, as the autocast GEMM's output);
//   2. the transfer (A, B) = (prod a, scan of b from 0) of each run of four
//      positions a lane holds; the two halves of the wave hold alternate runs
//      of one feature and swap them (v_permlane32_swap), so both compose the
//      128 positions of the wave in order; the wave with the first 128 rows
//      passes its transfer to the other through LDS;
//   3. the carry into the tile (the state before its first position): every
//      tile publishes its transfer as soon as it has it, and a
//      tile applies the published transfers of the tiles before it in the
//      sequence, in order, to the initial state;
//   4. every state from its run's carry, stepping h = a h + b through the run,
//      written as fp32 (and a bf16 copy for the next projection).
//
// The tiles are handed out by per-group tickets (an atomic counter per
// blockIdx % G group, tiles in position-major order within a group), so a
// workgroup only waits for tiles whose workgroups already hold lower tickets
// and are running, and those publish before they wait for anything: the
// waits always end. Every wait is also bounded: a transfer not seen after
// the spin limit (2^22 polls by default) sets a sticky status word to 1 and
// the tile's carry to NaN, so its states and everything computed from them
// are NaN, never silently wrong, and the caller learns of it from the status
// word; no launch can hang.
#include "common.hpp"
#include "mfma_stage.hpp"

namespace koemi {
namespace {

using mfma_stage::bf16x8;
using mfma_stage::f32x16;
using mfma_stage::kBK;
using mfma_stage::kOperandBytes;
using mfma_stage::slot_swizzle;
using mfma_stage::uniform_ptr;

constexpr int kGpRows = 256;  // positions per tile
constexpr int kGpThreads = mfma_stage::kThreads;
constexpr int kGpKAlign = 64;
constexpr int kGpWidthAlign = 128;  // features: a multiple of every tile width
constexpr uint32_t kSpinLimit = 1u << 22;
constexpr uint32_t kWithhold = 1u << 31;  // KOEMI_GP_WITHHOLD_TRANSFERS
constexpr int kMaxGroups = 8;

// Tile width: BNT B rows = BNT / 2 features (their retention rows, then their
// candidate rows). 256 (the default): 128 features, 256 accumulators per wave,
// one workgroup per CU. 128: 64 features, 128 accumulators per wave and two
// workgroups per CU (measured no faster at the C5 shape: the two workgroups
// of a CU run their phases in step, so one's epilogue does not hide under the
// other's main loop).
#ifndef KOEMI_GP_BN
#define KOEMI_GP_BN 256
#endif
constexpr int kGpBN = KOEMI_GP_BN;
static_assert(kGpBN == 128 || kGpBN == 256, "tile width");

// Workspace: kMaxGroups ticket counters (128 bytes apart) and the status word
// used when the caller passes none (word 256, byte offset 1024; 2 KiB in all,
// cleared to zero before every launch), then per tile and feature the
// published transfer as one 64-bit word (A in the low half, B in the high
// half), filled with kEmpty before every launch. A word is written once, by one
// 64-bit store, and read by 64-bit loads, so a reader sees either kEmpty or
// the whole pair: no flag and no fence is needed (an agent-scope fence would
// write back or invalidate the whole L2 of the XCD, under the operands of
// every other tile running there). kEmpty is two all-ones NaNs, which no gate
// arithmetic produces (NaNs it makes are canonical or carry a bf16 payload,
// whose low 16 bits are zero).
constexpr uint64_t kEmpty = ~uint64_t(0);
constexpr int64_t kCounterWords = 512;
struct GpWorkspace {
    size_t data_off, total;
};
// One transfer word per feature of every tile: batch x length / 256 x width.
inline GpWorkspace gp_workspace(int64_t batch, int64_t length, int64_t width) {
    GpWorkspace w;
    w.data_off = kCounterWords * sizeof(uint32_t);
    w.total = w.data_off + static_cast<size_t>(batch * (length / kGpRows) * width) * sizeof(uint64_t);
    return w;
}

// Zero the counter words, fill the transfer words with kEmpty.
__global__ void gp_clear_kernel(uint32_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = i < kCounterWords ? 0u : ~0u;
}

__device__ __forceinline__ float round_bf16(float x) { return static_cast<float>(static_cast<bf16>(x)); }

// (A, B) <- (A, B) then (a, b): h -> a (A h + B) + b.
__device__ __forceinline__ void then(float& A, float& B, float a, float b) {
    B = fmaf(a, B, b);
    A = A * a;
}

// The transfers of run q of m-tile mt of n-tile nt (retention accumulators
// nt, candidate nt + NT / 2, already turned into a and b): lo is the run of
// the wave's lower half (positions 8q .. 8q + 3 of the m-tile), hi the upper
// half's (8q + 4 .. 8q + 7), the same in both halves after the swap.
template <int NT>
__device__ __forceinline__ void run_transfer(const f32x16 (&acc)[4][NT], int nt, int mt, int q, float& loA, float& loB,
                                             float& hiA, float& hiB) {
    constexpr int NH = NT / 2;
    float A = acc[mt][nt][4 * q], B = acc[mt][nt + NH][4 * q];
#pragma unroll
    for (int i = 1; i < 4; ++i) then(A, B, acc[mt][nt][4 * q + i], acc[mt][nt + NH][4 * q + i]);
    const auto sa = __builtin_amdgcn_permlane32_swap(__float_as_uint(A), __float_as_uint(A), false, false);
    const auto sb = __builtin_amdgcn_permlane32_swap(__float_as_uint(B), __float_as_uint(B), false, false);
    loA = __uint_as_float(sa[0]);
    hiA = __uint_as_float(sa[1]);
    loB = __uint_as_float(sb[0]);
    hiB = __uint_as_float(sb[1]);
}

// One 256-position x BNT / 2-feature tile. Wave (wm, wn) holds positions
// wm * 128 .. + 127 and features wn * WF .. + WF - 1 of the tile (WF = BNT / 4):
// accumulators [m-tile][nt < NT / 2] are the retention pre-activations of
// features wn * WF + nt * 32 + lane % 32, [m-tile][nt + NT / 2] the candidate
// ones of the same features; element v of lane l is position mt * 32 +
// 8 (v / 4) + 4 (l / 32) + v % 4 of the wave's rows.
template <int BNT>
__global__ __launch_bounds__(kGpThreads, mfma_stage::TileShape<BNT>::kWgPerCu) void gated_projection_scan_kernel(
    const bf16* __restrict__ inputs, const bf16* __restrict__ weights, const bf16* __restrict__ biases,
    const uint8_t* __restrict__ valid, const float* __restrict__ initial, float* __restrict__ states,
    bf16* __restrict__ states16, int64_t s16_stride, float* __restrict__ final_states, int64_t L, int64_t F,
    int64_t K, int32_t n_ft, int32_t n_mt, int32_t groups, uint32_t* __restrict__ ws_words,
    uint64_t* __restrict__ ws_pairs, int32_t* __restrict__ status, uint32_t spin_limit) {
    using TS = mfma_stage::TileShape<BNT>;
    constexpr int NT = TS::kNT;  // n-tiles per wave
    constexpr int NH = NT / 2;   // of them retention (then as many candidate)
    constexpr int FEAT = BNT / 2;
    constexpr int WF = FEAT / 2;  // features per wave
    __shared__ __attribute__((aligned(1024))) char lds[TS::kStages * TS::kStageBytes];
    __shared__ float bias_sh[BNT];
    __shared__ uint8_t keep_sh[kGpRows];
    __shared__ float wave_sh[2][WF][2];     // the lower waves' transfers per feature (A, B)
    __shared__ float carry_sh[2][FEAT];     // the state before rows 0 and 128 of the tile
    __shared__ uint32_t ticket_sh;

    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;
    const int fl = lane & 31, hf = lane >> 5;

    // Ticket -> tile: group g = blockIdx % groups owns chains g * cg .. + cg - 1
    // (chain = sequence b x feature tile ft); tickets are position-major.
    const int32_t g = static_cast<int32_t>(blockIdx.x % static_cast<uint32_t>(groups));
    if (tid == 0) ticket_sh = atomicAdd(ws_words + g * 32, 1u);
    __syncthreads();
    const int32_t chains_g = (static_cast<int32_t>(gridDim.x) / n_mt) / groups;
    const int32_t ticket = static_cast<int32_t>(ticket_sh);
    const int32_t chain = g * chains_g + ticket % chains_g;
    const int32_t m = ticket / chains_g;
    const int32_t b = chain / n_ft, ft = chain % n_ft;
    const int64_t tix = static_cast<int64_t>(chain) * n_mt + m;
    const int64_t row0 = static_cast<int64_t>(b) * L + static_cast<int64_t>(m) * kGpRows;
    const int64_t n0 = static_cast<int64_t>(ft) * FEAT;

    // Stage copies (as the grouped GEMM's gate/value tile): A rows are the
    // tile's 256 positions; waves 0-1 copy the retention rows n0 .. n0 + FEAT
    // - 1, waves 2-3 the candidate rows F + n0 .. of the same features.
    const bf16* a_base = static_cast<const bf16*>(uniform_ptr(inputs + row0 * K));
    const bf16* b_base = static_cast<const bf16*>(uniform_ptr(weights + ((wave >= 2 ? F : 0) + n0) * K));
    uint32_t a_off[4], b_off[NT];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = (wave * 4 + i) * 16 + (lane >> 2);
        const int gk = (lane & 3) ^ slot_swizzle(r);
        a_off[i] = (static_cast<uint32_t>(r) * static_cast<uint32_t>(K) + gk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int r = (wave * NT + i) * 16 + (lane >> 2);
        const int gk = (lane & 3) ^ slot_swizzle(r);
        b_off[i] = (static_cast<uint32_t>(r & (FEAT - 1)) * static_cast<uint32_t>(K) + gk * 8) * 2u;
    }
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;
    const uint32_t a_lds = __builtin_amdgcn_readfirstlane(lds0 + wave * 4 * 1024);
    const uint32_t b_lds = __builtin_amdgcn_readfirstlane(lds0 + kOperandBytes + wave * NT * 1024);
    int a_row[4], b_row[NT];
#pragma unroll
    for (int t = 0; t < 4; ++t) a_row[t] = wm * 128 + t * 32 + fl;
#pragma unroll
    for (int t = 0; t < NT; ++t) b_row[t] = (t < NH ? wn * WF + t * 32 : FEAT + wn * WF + (t - NH) * 32) + fl;

    // Bias (thread t < FEAT: retention bias of feature n0 + t; FEAT <= t < BNT:
    // candidate bias of feature n0 + t - FEAT) and keep flag of position t,
    // read now so that their latency hides behind the main loop.
    float bias_mine = 0.0f;
    if (biases != nullptr && tid < BNT) bias_mine = to_f32(biases[tid < FEAT ? n0 + tid : F + n0 + tid - FEAT]);
    const uint8_t keep_mine = valid ? valid[row0 + tid] : uint8_t(1);

    f32x16 acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    mfma_stage::stage_loop<BNT, false>(lds, a_base, b_base, a_off, b_off, a_lds, b_lds, a_row, b_row, K / kBK, acc);

    if (tid < BNT) bias_sh[tid] = bias_mine;
    keep_sh[tid] = keep_mine;
    __syncthreads();

    // 1. Gates in place: acc[mt][nt] <- a, acc[mt][nt + NH] <- b (the keep flag
    // of a position serves its NH features).
    float br[NH], bc[NH];
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
        br[nt] = bias_sh[wn * WF + nt * 32 + fl];
        bc[nt] = bias_sh[FEAT + wn * WF + nt * 32 + fl];
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const bool keep = keep_sh[wm * 128 + mt * 32 + 8 * (v / 4) + 4 * hf + (v % 4)] != 0;
#pragma unroll
            for (int nt = 0; nt < NH; ++nt) {
                float a, bb;
                gate_pair(round_bf16(acc[mt][nt][v] + br[nt]), round_bf16(acc[mt][nt + NH][v] + bc[nt]), 0.0f, 0.0f,
                          keep, a, bb);
                acc[mt][nt][v] = a;
                acc[mt][nt + NH][v] = bb;
            }
        }
    }

    // 2. The wave's transfer over its 128 positions, per feature.
    float WA[NH], WB[NH];
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
        float A = 1.0f, B = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float loA, loB, hiA, hiB;
            run_transfer(acc, nt, j / 4, j % 4, loA, loB, hiA, hiB);
            then(A, B, loA, loB);
            then(A, B, hiA, hiB);
        }
        WA[nt] = A;
        WB[nt] = B;
    }
    if (wm == 0 && hf == 0) {
#pragma unroll
        for (int nt = 0; nt < NH; ++nt) {
            wave_sh[wn][nt * 32 + fl][0] = WA[nt];
            wave_sh[wn][nt * 32 + fl][1] = WB[nt];
        }
    }
    __syncthreads();

    // 3. The carry, by the upper waves: lane j < WF takes feature wn * WF + j
    // (n-tile j / 32, the half's own copy of the wave transfer).
    const int j = lane;
    if (wm == 1 && j < WF) {
        const float A0 = wave_sh[wn][j][0], B0 = wave_sh[wn][j][1];
        const float A1 = (NH == 2 && hf) ? WA[NH - 1] : WA[0], B1 = (NH == 2 && hf) ? WB[NH - 1] : WB[0];
        const float TA = A0 * A1, TB = fmaf(A1, B0, B1);  // the tile's transfer
        const int64_t feat = wn * WF + j;
        if (m + 1 < n_mt && !(spin_limit & kWithhold)) {  // the last tile's transfer is nobody's carry
            const uint64_t pair = static_cast<uint64_t>(__float_as_uint(TA)) |
                                  (static_cast<uint64_t>(__float_as_uint(TB)) << 32);
            __hip_atomic_store(ws_pairs + tix * FEAT + feat, pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // The carry: the initial state through the transfers of tiles 0 .. m - 1
        // in order (the same operations whatever the timing, so the states are
        // a deterministic function of the inputs).
        float C = initial[static_cast<int64_t>(b) * F + n0 + feat];
        const uint32_t limit = spin_limit & ~kWithhold;
        for (int32_t p = 0; p < m; ++p) {
            const uint64_t* src = ws_pairs + (static_cast<int64_t>(chain) * n_mt + p) * FEAT + feat;
            uint64_t pair;
            uint32_t spins = 0;
            while ((pair = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == kEmpty &&
                   spins < limit) {
                ++spins;
                __builtin_amdgcn_s_sleep(2);
            }
            if (pair == kEmpty) {  // timed out: report it, and poison the carry so no state is silently wrong
                __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                C = __builtin_nanf("");
                break;
            }
            C = fmaf(__uint_as_float(static_cast<uint32_t>(pair)), C, __uint_as_float(static_cast<uint32_t>(pair >> 32)));
        }
        carry_sh[0][feat] = C;
        carry_sh[1][feat] = fmaf(A0, C, B0);
    }
    __syncthreads();

    // 4. States: each run from its carry (composed from the wave's carry by
    // the run transfers in order), stepped through its four positions.
#pragma unroll
    for (int nt = 0; nt < NH; ++nt) {
        const int fi = wn * WF + nt * 32 + fl;
        const int64_t f = n0 + fi;
        float h = carry_sh[wm][fi];
#pragma unroll
        for (int jr = 0; jr < 16; ++jr) {
            const int mt = jr / 4, q = jr % 4;
            float loA, loB, hiA, hiB;
            run_transfer(acc, nt, mt, q, loA, loB, hiA, hiB);
            const float hmid = fmaf(loA, h, loB);
            float x = hf ? hmid : h;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int v = 4 * q + i;
                x = fmaf(acc[mt][nt][v], x, acc[mt][nt + NH][v]);
                const int64_t row = row0 + wm * 128 + mt * 32 + 8 * q + 4 * hf + i;
                states[row * F + f] = x;
                if (states16) states16[row * s16_stride + f] = static_cast<bf16>(x);
                // the sequence's last state, also on its own (the carried state)
                if (final_states && mt == 3 && q == 3 && i == 3 && hf == 1 && wm == 1 && m == n_mt - 1)
                    final_states[static_cast<int64_t>(b) * F + f] = x;
            }
            h = fmaf(hiA, hmid, hiB);
        }
    }
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" size_t koemi_gated_projection_scan_workspace_bytes(int64_t batch, int64_t length, int64_t width) {
    if (batch <= 0 || length <= 0 || width <= 0 || length % kGpRows || width % kGpWidthAlign) return 0;
    return gp_workspace(batch, length, width).total;
}

extern "C" int koemi_gated_projection_scan(const void* inputs, const void* weights, const void* biases,
                                           const uint8_t* valid, const float* initial, float* states,
                                           void* states_bf16, int64_t bf16_row_stride, float* final_states,
                                           int64_t batch,
                                           int64_t length, int64_t width, int64_t input_width, void* workspace,
                                           size_t workspace_bytes, int32_t* status, uint32_t spin_limit,
                                           koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1 || input_width < 1)
        return fail(KOEMI_ERR_INVALID, "gated projection scan needs non-negative batch and length and positive widths");
    if (length % kGpRows || width % kGpWidthAlign || input_width % kGpKAlign)
        return fail(KOEMI_ERR_UNSUPPORTED,
                    "gated projection scan needs length %% %d == 0, width %% %d == 0 and input width %% %d == 0 "
                    "(got %lld, %lld, %lld)",
                    kGpRows, kGpWidthAlign, kGpKAlign, static_cast<long long>(length), static_cast<long long>(width),
                    static_cast<long long>(input_width));
    if (batch * length == 0) return KOEMI_OK;
    if (!inputs || !weights || !initial || !states || !workspace)
        return fail(KOEMI_ERR_INVALID, "gated projection scan received a null pointer");
    if ((reinterpret_cast<uintptr_t>(inputs) | reinterpret_cast<uintptr_t>(weights)) & 15)
        return fail(KOEMI_ERR_UNSUPPORTED, "gated projection scan needs 16-byte aligned inputs and weights");
    if (bf16_row_stride == 0) bf16_row_stride = width;
    if (states_bf16 != nullptr && bf16_row_stride < width)
        return fail(KOEMI_ERR_INVALID, "gated projection scan: the bf16 row stride is below the width");
    const int64_t n_mt = length / kGpRows, n_ft = width / (kGpBN / 2);
    const int64_t chains = batch * n_ft, tiles = chains * n_mt;
    if (tiles > 0x7fffffffLL || input_width > (1LL << 22) || width > (1LL << 20))
        return fail(KOEMI_ERR_UNSUPPORTED, "gated projection scan shape too large");
    const GpWorkspace w = gp_workspace(batch, length, width);
    if (workspace_bytes < w.total)
        return fail(KOEMI_ERR_INVALID, "gated projection scan workspace too small: need %zu bytes", w.total);
    int groups = kMaxGroups;
    while (chains % groups) groups /= 2;
    hipStream_t s = as_stream(stream);
    uint32_t* words = static_cast<uint32_t*>(workspace);
    const int64_t clear_words = static_cast<int64_t>(w.total / sizeof(uint32_t));
    hipLaunchKernelGGL(gp_clear_kernel, dim3(static_cast<uint32_t>((clear_words + 255) / 256)), dim3(256), 0, s, words,
                       clear_words);
    if (int st = check_launch("gated projection scan (clear)")) return st;
    hipLaunchKernelGGL(gated_projection_scan_kernel<kGpBN>, dim3(static_cast<uint32_t>(tiles)), dim3(kGpThreads), 0, s,
                       static_cast<const bf16*>(inputs), static_cast<const bf16*>(weights),
                       static_cast<const bf16*>(biases), valid, initial, states, static_cast<bf16*>(states_bf16),
                       bf16_row_stride, final_states, length, width, input_width, static_cast<int32_t>(n_ft),
                       static_cast<int32_t>(n_mt), static_cast<int32_t>(groups), words,
                       reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + w.data_off),
                       status ? status : reinterpret_cast<int32_t*>(words + kMaxGroups * 32),
                       (spin_limit & ~kWithhold) ? spin_limit : (spin_limit | kSpinLimit));
    return check_launch("gated projection scan");
}
