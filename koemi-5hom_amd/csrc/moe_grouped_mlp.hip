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

namespace koemi {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kPad = 8;  // bf16 elements of row padding in LDS (conflict-free 16 B fragment reads)
constexpr int kLdsStride = kBK + kPad;
constexpr int kGemmThreads = 256;

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

struct MlpWorkspace {
    size_t hidden_off, slot_expert_off, slot_row_off, slot_end_off, total;
    int64_t max_slots;
};

// The MFMA path (both GEMM K dimensions multiples of kBK) keeps H in bf16; the
// SIMT path keeps it in fp32.
inline bool mfma_shape(int64_t width, int64_t hidden, int dtype) {
    return dtype == KOEMI_BF16 && width % kBK == 0 && hidden % kBK == 0;
}

inline MlpWorkspace mlp_workspace(int64_t pairs, int64_t width, int64_t hidden, int64_t E, int dtype) {
    MlpWorkspace w;
    w.max_slots = (pairs + kBM - 1) / kBM + E;
    const size_t elem = mfma_shape(width, hidden, dtype) ? 2 : 4;
    w.hidden_off = 0;
    w.slot_expert_off = align256(static_cast<size_t>(pairs > 0 ? pairs : 1) * static_cast<size_t>(hidden) * elem);
    w.slot_row_off = w.slot_expert_off + align256(static_cast<size_t>(w.max_slots) * sizeof(int32_t));
    w.slot_end_off = w.slot_row_off + align256(static_cast<size_t>(w.max_slots) * sizeof(int64_t));
    w.total = w.slot_end_off + align256(static_cast<size_t>(w.max_slots) * sizeof(int64_t));
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
    __shared__ int32_t span_sum[kSchedThreads];
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
    span_sum[tid] = sum;
    __syncthreads();
    if (tid == 0) {
        int32_t run = 0;
        for (int i = 0; i < kSchedThreads; ++i) {
            const int32_t v = span_sum[i];
            span_sum[i] = run;
            run += v;
        }
    }
    __syncthreads();
    int32_t run = span_sum[tid];
    for (int64_t e = b0; e < b1; ++e) {
        const int32_t v = first_tile[e];
        first_tile[e] = run;
        run += v;
    }
    __syncthreads();
    const int64_t total = first_tile[E];
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

// One 128x128 output tile (GLU: 128 rows x 64 hidden units) per workgroup; four
// waves in a 2x2 arrangement, each owning 64 rows x 64 B-rows as 2x2 MFMA
// 32x32 tiles. The next K tile is fetched into registers while the current one
// is multiplied out of LDS.
template <bool GLU>
__global__ __launch_bounds__(kGemmThreads) void grouped_gemm_bf16_kernel(
    const bf16* __restrict__ A, const bf16* __restrict__ W0, const bf16* __restrict__ W1,
    const bf16* __restrict__ bias0, const bf16* __restrict__ bias1, bf16* __restrict__ C,
    const int32_t* __restrict__ slot_expert, const int64_t* __restrict__ slot_row,
    const int64_t* __restrict__ slot_end, int64_t n_out, int64_t K) {
    __shared__ __attribute__((aligned(16))) bf16 As[kBM * kLdsStride];
    __shared__ __attribute__((aligned(16))) bf16 Bs[kBN * kLdsStride];

    const int e = slot_expert[blockIdx.x];
    if (e < 0) return;
    const int64_t row0 = slot_row[blockIdx.x];
    const int64_t row_end = slot_end[blockIdx.x];
    const int tid = threadIdx.x;
    const int lane = lane_id();
    const int wave = tid / kWave;
    const int wm = wave >> 1, wn = wave & 1;

    // B rows of this tile: GLU -> 64 gate rows then 64 value rows of hidden units
    // [h0, h0 + 64); plain -> 128 consecutive output columns from n0.
    const int64_t n0 = GLU ? static_cast<int64_t>(blockIdx.y) * (kBN / 2) : static_cast<int64_t>(blockIdx.y) * kBN;
    const bf16* We0 = W0 + static_cast<int64_t>(e) * n_out * K;
    const bf16* We1 = GLU ? W1 + static_cast<int64_t>(e) * n_out * K : nullptr;

    // Global load assignment: 4 16-byte chunks of A and 4 of B per thread. The
    // loads are unconditional at clamped addresses (a branch around a load would
    // make the compiler wait for the prefetch too); rows past the segment or the
    // output width only feed discarded outputs. K is a multiple of kBK.
    uint4 ra[4], rb[4];
    auto load_tiles = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * kGemmThreads;
            const int r = c >> 3, cc = (c & 7) * 8;
            const int64_t kc = k0 + cc;
            const int64_t grow = min(row0 + r, row_end - 1);
            ra[i] = *reinterpret_cast<const uint4*>(A + grow * K + kc);
            const bf16* src = (GLU && r >= 64) ? We1 : We0;
            const int64_t n = min(GLU ? n0 + (r & 63) : n0 + r, n_out - 1);
            rb[i] = *reinterpret_cast<const uint4*>(src + n * K + kc);
        }
    };
    auto store_tiles = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * kGemmThreads;
            const int r = c >> 3, cc = (c & 7) * 8;
            *reinterpret_cast<uint4*>(As + r * kLdsStride + cc) = ra[i];
            *reinterpret_cast<uint4*>(Bs + r * kLdsStride + cc) = rb[i];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // B-row base of each of the wave's two n-tiles.
    int brow[2];
    if (GLU) {
        brow[0] = wn * 32;       // gate rows of hidden units h0 + wn*32 ...
        brow[1] = 64 + wn * 32;  // value rows of the same hidden units
    } else {
        brow[0] = wn * 64;
        brow[1] = wn * 64 + 32;
    }
    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 8;

    load_tiles(0);
    for (int64_t k0 = 0; k0 < K; k0 += kBK) {
        store_tiles();
        __syncthreads();
        if (k0 + kBK < K) load_tiles(k0 + kBK);
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 16) {
            bf16x8 af[2], bfr[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
                af[mt] = *reinterpret_cast<const bf16x8*>(As + (wm * 64 + mt * 32 + frag_row) * kLdsStride + kk + frag_k);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
                bfr[nt] = *reinterpret_cast<const bf16x8*>(Bs + (brow[nt] + frag_row) * kLdsStride + kk + frag_k);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mt], bfr[nt], acc[mt][nt], 0, 0, 0);
        }
        __syncthreads();
    }

    // Epilogue. Accumulator element v of lane l is row (l/32)*4 + v%4 + (v/4)*8,
    // column l%32 of its 32x32 tile.
    const int col_in_tile = lane & 31;
    const int row_base = (lane >> 5) * 4;
    if (GLU) {
        const int64_t h = n0 + wn * 32 + col_in_tile;
        if (h < n_out) {
            const float bg = to_f32(bias0[static_cast<int64_t>(e) * n_out + h]);
            const float bv = to_f32(bias1[static_cast<int64_t>(e) * n_out + h]);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t grow = row0 + wm * 64 + mt * 32 + row_base + (v & 3) + (v >> 2) * 8;
                    if (grow < row_end) {
                        const float g = acc[mt][0][v] + bg;
                        const float u = acc[mt][1][v] + bv;
                        C[grow * n_out + h] = from_f32<bf16>(silu_f(g) * u);
                    }
                }
        }
    } else {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int64_t col = n0 + wn * 64 + nt * 32 + col_in_tile;
            if (col >= n_out) continue;
            const float bo = to_f32(bias0[static_cast<int64_t>(e) * n_out + col]);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t grow = row0 + wm * 64 + mt * 32 + row_base + (v & 3) + (v >> 2) * 8;
                    if (grow < row_end) C[grow * n_out + col] = from_f32<bf16>(acc[mt][nt][v] + bo);
                }
        }
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

int run_mfma(const void* x, const int64_t* offsets, const void* Wg, const void* bg, const void* Wv, const void* bv,
             const void* Wo, const void* bo, void* y, int64_t P, int64_t D, int64_t Hd, int64_t E,
             const MlpWorkspace& ws, char* base, hipStream_t s) {
    bf16* H = reinterpret_cast<bf16*>(base + ws.hidden_off);
    int32_t* slot_expert = reinterpret_cast<int32_t*>(base + ws.slot_expert_off);
    int64_t* slot_row = reinterpret_cast<int64_t*>(base + ws.slot_row_off);
    int64_t* slot_end = reinterpret_cast<int64_t*>(base + ws.slot_end_off);
    if (ws.max_slots > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many tiles");
    if (E > kMaxScheduleExperts) return fail(KOEMI_ERR_UNSUPPORTED, "grouped MLP supports at most %lld experts",
                                             static_cast<long long>(kMaxScheduleExperts));
    hipLaunchKernelGGL(build_schedule_kernel, dim3(1), dim3(kSchedThreads), static_cast<size_t>(E + 1) * sizeof(int32_t),
                       s, offsets, E, P, ws.max_slots, slot_expert, slot_row, slot_end);
    int st = check_launch("koemi_moe_grouped_mlp(schedule)");
    if (st != KOEMI_OK) return st;
    const unsigned slots = static_cast<unsigned>(ws.max_slots);
    hipLaunchKernelGGL((grouped_gemm_bf16_kernel<true>), dim3(slots, grid_for(Hd, kBN / 2)), dim3(kGemmThreads), 0, s,
                       static_cast<const bf16*>(x), static_cast<const bf16*>(Wg), static_cast<const bf16*>(Wv),
                       static_cast<const bf16*>(bg), static_cast<const bf16*>(bv), H, slot_expert, slot_row, slot_end, Hd, D);
    st = check_launch("koemi_moe_grouped_mlp(gemm1)");
    if (st != KOEMI_OK) return st;
    hipLaunchKernelGGL((grouped_gemm_bf16_kernel<false>), dim3(slots, grid_for(D, kBN)), dim3(kGemmThreads), 0, s, H,
                       static_cast<const bf16*>(Wo), nullptr, static_cast<const bf16*>(bo), nullptr,
                       static_cast<bf16*>(y), slot_expert, slot_row, slot_end, D, Hd);
    st = check_launch("koemi_moe_grouped_mlp(gemm2)");
    if (st != KOEMI_OK) return st;
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
                         reinterpret_cast<uintptr_t>(output_weights) % 16 == 0;
    if (mfma_shape(width, hidden, dtype) && !aligned)
        return fail(KOEMI_ERR_INVALID, "grouped MLP bf16 operands must be 16-byte aligned");
    if (mfma_shape(width, hidden, dtype))
        return run_mfma(sorted_context, segment_offsets, gate_weights, gate_biases, value_weights, value_biases,
                        output_weights, output_biases, output, pairs, width, hidden, expert_count, ws, base, s);
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
