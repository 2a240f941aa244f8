// Deterministic MoE combine for gfx950.
//
// Reference: cuda_kernels/moe/moe_kernels.cu:201-229, 560-582 — fp32 atomicAdd
// of y / top_k into a zeroed fp32 [tokens, width] buffer, then a cast. That
// costs a zero-fill, read-modify-write atomics and a cast pass, and the sum
// order depends on scheduling for top_k > 2. Here:
//
//   1. invert sorted_rows: each valid sorted position i records itself under
//      its token (one int atomic per pair, used only to claim a slot);
//   2. one wave per token sorts its (at most top_k) positions ascending, sums
//      y_i * w_i in fp32 in that order and writes the row once in the output
//      dtype.
//
// HBM traffic is one read of every valid expert output row and one write of
// every token row.
#include "common.hpp"

namespace koemi {
namespace {

constexpr int kCombineWaves = 4;
constexpr int kMaxTopK = 256;

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

__global__ void zero_i32_kernel(int32_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// Steps 1 for a small combine (a decode step) in one workgroup: the
// per-token counters live in LDS, so no separate zero-fill runs.
constexpr int kSmallInvertTokens = 8192;
__global__ __launch_bounds__(1024) void invert_rows_small_kernel(const int64_t* __restrict__ sorted_rows,
                                                                 const int64_t* __restrict__ valid_end,
                                                                 int32_t* __restrict__ cnt, int64_t* __restrict__ pos,
                                                                 int64_t pairs, int64_t tokens, int64_t k) {
    __shared__ int32_t c_sh[kSmallInvertTokens];
    for (int64_t t = threadIdx.x; t < tokens; t += 1024) c_sh[t] = 0;
    __syncthreads();
    const int64_t valid = min(*valid_end, pairs);
    for (int64_t i = threadIdx.x; i < valid; i += 1024) {
        const int64_t t = sorted_rows[i];
        if (t < 0 || t >= tokens) continue;
        const int32_t slot = atomicAdd(&c_sh[t], 1);
        if (slot < k) pos[t * k + slot] = i;
    }
    __syncthreads();
    for (int64_t t = threadIdx.x; t < tokens; t += 1024) cnt[t] = c_sh[t];
}

__global__ void invert_rows_kernel(const int64_t* __restrict__ sorted_rows, const int64_t* __restrict__ valid_end,
                                   int32_t* __restrict__ cnt, int64_t* __restrict__ pos, int64_t pairs, int64_t tokens,
                                   int64_t k) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t valid = min(*valid_end, pairs);
    if (i >= valid) return;
    const int64_t t = sorted_rows[i];
    if (t < 0 || t >= tokens) return;
    const int32_t slot = atomicAdd(&cnt[t], 1);
    if (slot < k) pos[t * k + slot] = i;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kWave * kCombineWaves) void combine_rows_kernel(
    const T* __restrict__ y, const int32_t* __restrict__ cnt, const int64_t* __restrict__ pos,
    const float* __restrict__ pair_w, T* __restrict__ out, int64_t tokens, int64_t k, int64_t D) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kCombineWaves + threadIdx.x / kWave;
    if (t >= tokens) return;
    const int lane = lane_id();
    const int n = min(static_cast<int64_t>(cnt[t]), k);
    const int64_t* mine = pos + t * k;
    const float inv_k_div = static_cast<float>(k);
    if constexpr (VEC) {
        constexpr int N = 16 / sizeof(T);
        union V {
            uint4 raw;
            T e[N];
        };
        const int64_t nvec = D / N;
        for (int64_t v0 = 0; v0 < nvec; v0 += 2 * kWave) {
            float acc[2][N];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int q = 0; q < N; ++q) acc[u][q] = 0.0f;
            int64_t last = -1;
            for (int r = 0; r < n; ++r) {
                // r-th smallest position of this token (n <= k, k small).
                int64_t best = INT64_MAX;
                for (int j = 0; j < n; ++j) {
                    const int64_t pj = mine[j];
                    if (pj > last && pj < best) best = pj;
                }
                last = best;
                const float w = pair_w ? pair_w[best] : 0.0f;
                const T* row = y + best * D;
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int64_t v = v0 + u * kWave + lane;
                    if (v < nvec) {
                        V in;
                        in.raw = reinterpret_cast<const uint4*>(row)[v];
#pragma unroll
                        for (int q = 0; q < N; ++q) {
                            const float f = to_f32(in.e[q]);
                            acc[u][q] += pair_w ? f * w : f / inv_k_div;
                        }
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int64_t v = v0 + u * kWave + lane;
                if (v < nvec) {
                    V o;
#pragma unroll
                    for (int q = 0; q < N; ++q) o.e[q] = from_f32<T>(acc[u][q]);
                    reinterpret_cast<uint4*>(out + t * D)[v] = o.raw;
                }
            }
        }
    } else {
        for (int64_t c = lane; c < D; c += kWave) {
            float acc = 0.0f;
            int64_t last = -1;
            for (int r = 0; r < n; ++r) {
                int64_t best = INT64_MAX;
                for (int j = 0; j < n; ++j) {
                    const int64_t pj = mine[j];
                    if (pj > last && pj < best) best = pj;
                }
                last = best;
                const float f = to_f32(y[best * D + c]);
                acc += pair_w ? f * pair_w[best] : f / inv_k_div;
            }
            out[t * D + c] = from_f32<T>(acc);
        }
    }
}

// top_k <= KMAX: the token's positions live in registers, sorted ascending by
// a compare-exchange network, and every row load of a vector step is issued
// before the first add (loads are unconditional at clamped addresses; rows
// beyond the token's count reuse its first row and are skipped in the sum).
template <int KMAX>
__device__ __forceinline__ void sort_positions(int64_t (&p)[KMAX]) {
#pragma unroll
    for (int i = 0; i < KMAX; ++i)
#pragma unroll
        for (int j = 0; j + 1 < KMAX - i; ++j) {
            const int64_t lo = min(p[j], p[j + 1]), hi = max(p[j], p[j + 1]);
            p[j] = lo;
            p[j + 1] = hi;
        }
}

template <typename T, int KMAX, bool VEC, bool NTS = false>
__global__ __launch_bounds__(kWave * kCombineWaves) void combine_rows_small_kernel(
    const T* __restrict__ y, const int32_t* __restrict__ cnt, const int64_t* __restrict__ pos,
    const float* __restrict__ pair_w, T* __restrict__ out, int64_t tokens, int64_t k, int64_t D) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kCombineWaves + threadIdx.x / kWave;
    if (t >= tokens) return;
    const int lane = lane_id();
    const int n = static_cast<int>(min(static_cast<int64_t>(cnt[t]), k));
    int64_t p[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        const int64_t pj = pos[t * k + min(static_cast<int64_t>(j), k - 1)];
        p[j] = j < n ? pj : INT64_MAX;
    }
    sort_positions<KMAX>(p);
    const float kf = static_cast<float>(k);
    T* orow = out + t * D;
    if (n == 0) {
        for (int64_t c = lane; c < D; c += kWave) orow[c] = from_f32<T>(0.0f);
        return;
    }
    const T* rows[KMAX];
    float w[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        const int64_t pj = j < n ? p[j] : p[0];
        rows[j] = y + pj * D;
        w[j] = pair_w ? pair_w[pj] : 0.0f;
    }
    if constexpr (VEC) {
        constexpr int N = 16 / sizeof(T);
        union V {
            uint4 raw;
            T e[N];
        };
        const int64_t nvec = D / N;
        for (int64_t v0 = 0; v0 < nvec; v0 += kWave) {
            const int64_t v = v0 + lane;
            const int64_t vc = v < nvec ? v : nvec - 1;
            V in[KMAX];
#pragma unroll
            for (int j = 0; j < KMAX; ++j) in[j].raw = reinterpret_cast<const uint4*>(rows[j])[vc];
            float acc[N];
#pragma unroll
            for (int q = 0; q < N; ++q) acc[q] = 0.0f;
#pragma unroll
            for (int j = 0; j < KMAX; ++j) {
                if (j < n) {
#pragma unroll
                    for (int q = 0; q < N; ++q) {
                        const float f = to_f32(in[j].e[q]);
                        acc[q] += pair_w ? f * w[j] : f / kf;
                    }
                }
            }
            if (v < nvec) {
                V o;
#pragma unroll
                for (int q = 0; q < N; ++q) o.e[q] = from_f32<T>(acc[q]);
                if constexpr (NTS) store16_nt(reinterpret_cast<uint4*>(orow) + v, o.raw);
                else reinterpret_cast<uint4*>(orow)[v] = o.raw;
            }
        }
    } else {
        for (int64_t c0 = 0; c0 < D; c0 += kWave) {
            const int64_t c = c0 + lane;
            const int64_t cc = c < D ? c : D - 1;
            float in[KMAX];
#pragma unroll
            for (int j = 0; j < KMAX; ++j) in[j] = to_f32(rows[j][cc]);
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < KMAX; ++j)
                if (j < n) acc += pair_w ? in[j] * w[j] : in[j] / kf;
            if (c < D) orow[c] = from_f32<T>(acc);
        }
    }
}

struct CombineWorkspace {
    size_t cnt_off, pos_off, total;
};
inline CombineWorkspace combine_workspace(int64_t tokens, int64_t k) {
    CombineWorkspace w;
    w.cnt_off = 0;
    w.pos_off = align256(static_cast<size_t>(tokens) * sizeof(int32_t));
    w.total = w.pos_off + align256(static_cast<size_t>(tokens) * static_cast<size_t>(k) * sizeof(int64_t));
    return w;
}

template <typename T>
int launch_combine_rows(const void* y, const int32_t* cnt, const int64_t* pos, const float* pair_w, void* out,
                        int64_t tokens, int64_t k, int64_t D, hipStream_t s) {
    const bool vec = (D * static_cast<int64_t>(sizeof(T))) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const dim3 grid(grid_for(tokens, kCombineWaves)), block(kWave * kCombineWaves);
    const bool nts = tokens * D * static_cast<int64_t>(sizeof(T)) > KOEMI_NT_STORE_BYTES;  // written once, far beyond the caches
#define KOEMI_COMBINE_SMALL(KMAX)                                                                                   \
    if (k <= KMAX) {                                                                                                \
        if (vec && nts)                                                                                             \
            hipLaunchKernelGGL((combine_rows_small_kernel<T, KMAX, true, true>), grid, block, 0, s,                 \
                               static_cast<const T*>(y), cnt, pos, pair_w, static_cast<T*>(out), tokens, k, D);      \
        else if (vec)                                                                                               \
            hipLaunchKernelGGL((combine_rows_small_kernel<T, KMAX, true>), grid, block, 0, s,                       \
                               static_cast<const T*>(y), cnt, pos, pair_w, static_cast<T*>(out), tokens, k, D);      \
        else                                                                                                        \
            hipLaunchKernelGGL((combine_rows_small_kernel<T, KMAX, false>), grid, block, 0, s,                      \
                               static_cast<const T*>(y), cnt, pos, pair_w, static_cast<T*>(out), tokens, k, D);      \
        return check_launch("koemi_moe_combine(rows)");                                                             \
    }
    KOEMI_COMBINE_SMALL(2)
    KOEMI_COMBINE_SMALL(4)
    KOEMI_COMBINE_SMALL(8)
#undef KOEMI_COMBINE_SMALL
    if (vec)
        hipLaunchKernelGGL((combine_rows_kernel<T, true>), grid, block, 0, s, static_cast<const T*>(y), cnt, pos, pair_w,
                           static_cast<T*>(out), tokens, k, D);
    else
        hipLaunchKernelGGL((combine_rows_kernel<T, false>), grid, block, 0, s, static_cast<const T*>(y), cnt, pos, pair_w,
                           static_cast<T*>(out), tokens, k, D);
    return check_launch("koemi_moe_combine(rows)");
}

// The HERM block's expert tail in one pass per token row (a wave per row):
// the combine above (the k expert outputs in ascending sorted position, each
// scaled by its weight or by 1/k, summed in fp32 from zero and rounded once to
// bf16: combine_topk), the expert output normalizer with the residual and the
// valid-row select (RMSNorm of context + update, rows whose mask is false keep
// the context: experts.py:134-136, layers.py:14-16) and, with w_next, the next
// block's input RMSNorm of that result (network.py:296-310), each step with
// the arithmetic of the separate kernels it replaces (the same bits): lane l
// holds columns (j * 64 + l) * 4 .. + 3, j < NV; the sum of squares runs in
// (j, i) order per lane, then over the lanes by xor butterfly.
// POS: pos holds every pair's sorted position (the permutation's own
// pair -> position map, k per token; a pair is valid when its position is
// below *valid_end) and cnt is unused; otherwise cnt / pos come from the
// inversion above (the first cnt[t] entries of the token's row).
// PRE (a decode step's few rows): the row's context and both norm weights
// are loaded first, ahead of the pair-position chain they do not depend on;
// many rows (a prefill) load them where they are used, which keeps the
// registers, and the occupancy, of a bandwidth-bound pass.
// FN: the context is not read; it is the fusion normalizer's output
// RMSNorm(fusion) * w_fusion (network.py:723-732), formed here from the bf16
// fusion rows with the arithmetic of herm_rmsnorm_kernel (the same lanes,
// the same sum-of-squares order: the same bits as the fp32 rows that kernel
// writes), so that no fp32 copy of it goes through memory.
template <int KMAX, int NV, bool POS, bool PRE = false, bool FN = false>
__global__ __launch_bounds__(kWave * kCombineWaves) void combine_norm_kernel(
    const bf16* __restrict__ y, const int32_t* __restrict__ cnt, const int64_t* __restrict__ pos,
    const int64_t* __restrict__ valid_end, const float* __restrict__ pair_w, const float* __restrict__ ctx,
    const uint8_t* __restrict__ mask, const float* __restrict__ w_expert, const float* __restrict__ w_next,
    float* __restrict__ out, bf16* __restrict__ out_next, int64_t tokens, int64_t k, int H, float eps,
    const bf16* __restrict__ fusion, const float* __restrict__ w_fusion) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kCombineWaves + threadIdx.x / kWave;
    if (t >= tokens) return;
    const int lane = lane_id();
    const float* xr = ctx + t * H;
    float4 xq[NV], wq_e[NV], wq_n[NV];
    if constexpr (FN) {
        float fv[NV][4];
        float ssf = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = (j * kWave + lane) * 4;
            if (c < H) {
                const float4 q = load4(fusion + t * H + c);
                fv[j][0] = q.x; fv[j][1] = q.y; fv[j][2] = q.z; fv[j][3] = q.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) fv[j][i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) ssf = fmaf(fv[j][i], fv[j][i], ssf);
        }
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) ssf += __shfl_xor(ssf, off, kWave);
        const float invf = rsqrtf(ssf / static_cast<float>(H) + eps);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = (j * kWave + lane) * 4;
            const float4 wq = *reinterpret_cast<const float4*>(w_fusion + (c < H ? c : 0));
            xq[j] = make_float4(fv[j][0] * invf * wq.x, fv[j][1] * invf * wq.y, fv[j][2] * invf * wq.z,
                                fv[j][3] * invf * wq.w);
        }
    }
    if constexpr (PRE) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int c = (j * kWave + lane) * 4;
            const int cc = c < H ? c : 0;
            if constexpr (!FN) xq[j] = *reinterpret_cast<const float4*>(xr + cc);
            wq_e[j] = *reinterpret_cast<const float4*>(w_expert + cc);
            wq_n[j] = w_next != nullptr ? *reinterpret_cast<const float4*>(w_next + cc)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    auto ctx4 = [&](int j, int c) { return (PRE || FN) ? xq[j] : *reinterpret_cast<const float4*>(xr + c); };
    auto we4 = [&](int j, int c) { return PRE ? wq_e[j] : *reinterpret_cast<const float4*>(w_expert + c); };
    auto wn4 = [&](int j, int c) { return PRE ? wq_n[j] : *reinterpret_cast<const float4*>(w_next + c); };
    int n = 0;
    int64_t p[KMAX];
    if constexpr (POS) {
        const int64_t end = *valid_end;
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            const int64_t pj = j < k ? pos[t * k + j] : INT64_MAX;
            const bool ok = pj >= 0 && pj < end;
            p[j] = ok ? pj : INT64_MAX;
            n += ok ? 1 : 0;
        }
    } else {
        n = static_cast<int>(min(static_cast<int64_t>(cnt[t]), k));
#pragma unroll
        for (int j = 0; j < KMAX; ++j) {
            const int64_t pj = pos[t * k + min(static_cast<int64_t>(j), k - 1)];
            p[j] = j < n ? pj : INT64_MAX;
        }
    }
    sort_positions<KMAX>(p);
    const float kf = static_cast<float>(k);
    float w[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) w[j] = (pair_w != nullptr && j < n) ? pair_w[p[j]] : 0.0f;
    float v[NV][4];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * kWave + lane) * 4;
        if (c < H) {
            const float4 q = ctx4(j, c);
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < KMAX; ++m) {
                if (m < n) {
                    const float4 e = load4(y + p[m] * H + c);
                    const float ev[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] += pair_w ? ev[i] * w[m] : ev[i] / kf;
                }
            }
            v[j][0] = q.x + to_f32(from_f32<bf16>(acc[0]));
            v[j][1] = q.y + to_f32(from_f32<bf16>(acc[1]));
            v[j][2] = q.z + to_f32(from_f32<bf16>(acc[2]));
            v[j][3] = q.w + to_f32(from_f32<bf16>(acc[3]));
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[j][i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) ss = fmaf(v[j][i], v[j][i], ss);
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
    const bool keep = mask == nullptr || mask[t] != 0;
    const float inv = rsqrtf(ss / static_cast<float>(H) + eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * kWave + lane) * 4;
        if (c >= H) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[j][i] = 0.0f;
        } else if (keep) {
            const float4 wq = we4(j, c);
            v[j][0] = v[j][0] * inv * wq.x;
            v[j][1] = v[j][1] * inv * wq.y;
            v[j][2] = v[j][2] * inv * wq.z;
            v[j][3] = v[j][3] * inv * wq.w;
        } else {
            const float4 q = ctx4(j, c);
            v[j][0] = q.x; v[j][1] = q.y; v[j][2] = q.z; v[j][3] = q.w;
        }
        if (out != nullptr && c < H) *reinterpret_cast<float4*>(out + t * H + c) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
#pragma unroll
        for (int i = 0; i < 4; ++i) ss2 = fmaf(v[j][i], v[j][i], ss2);
    }
    if (w_next == nullptr || out_next == nullptr) return;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) ss2 += __shfl_xor(ss2, off, kWave);
    const float inv2 = rsqrtf(ss2 / static_cast<float>(H) + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c = (j * kWave + lane) * 4;
        if (c >= H) continue;
        const float4 wq = wn4(j, c);
        typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
        bf16x4 q;
        q[0] = static_cast<__bf16>(v[j][0] * inv2 * wq.x);
        q[1] = static_cast<__bf16>(v[j][1] * inv2 * wq.y);
        q[2] = static_cast<__bf16>(v[j][2] * inv2 * wq.z);
        q[3] = static_cast<__bf16>(v[j][3] * inv2 * wq.w);
        *reinterpret_cast<bf16x4*>(out_next + t * H + c) = q;
    }
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" size_t koemi_moe_combine_workspace_bytes(int64_t tokens, int64_t top_k) {
    if (tokens < 1 || top_k < 1) return 0;
    return combine_workspace(tokens, top_k).total;
}

extern "C" int koemi_moe_combine(const void* expert_outputs, const int64_t* sorted_rows,
                                 const int64_t* segment_offsets, const float* pair_weights, void* combined,
                                 int64_t pairs, int64_t width, int64_t tokens, int64_t top_k, int64_t num_segments,
                                 int dtype, void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (tokens < 1 || width < 1 || pairs < 0) return fail(KOEMI_ERR_INVALID, "combine needs tokens >= 1, width >= 1");
    if (top_k < 1 || top_k > kMaxTopK) return fail(KOEMI_ERR_INVALID, "top_k must be in [1, %d]", kMaxTopK);
    if (num_segments < 1) return fail(KOEMI_ERR_INVALID, "segment_offsets must have at least two entries");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "combine does not support dtype %s", dtype_name(dtype));
    if (!segment_offsets || !combined || (pairs > 0 && (!expert_outputs || !sorted_rows)))
        return fail(KOEMI_ERR_INVALID, "combine received a null pointer");
    const CombineWorkspace ws = combine_workspace(tokens, top_k);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "combine workspace too small: need %zu bytes", ws.total);
    char* base = static_cast<char*>(workspace);
    int32_t* cnt = reinterpret_cast<int32_t*>(base + ws.cnt_off);
    int64_t* pos = reinterpret_cast<int64_t*>(base + ws.pos_off);
    hipStream_t s = as_stream(stream);
    int st = KOEMI_OK;
    if (tokens <= kSmallInvertTokens && pairs <= 4096) {
        hipLaunchKernelGGL(invert_rows_small_kernel, dim3(1), dim3(1024), 0, s, sorted_rows,
                           segment_offsets + num_segments, cnt, pos, pairs, tokens, top_k);
        st = check_launch("koemi_moe_combine(invert)");
        if (st != KOEMI_OK) return st;
    } else {
        hipLaunchKernelGGL(zero_i32_kernel, dim3(grid_for(tokens, 256)), dim3(256), 0, s, cnt, tokens);
        st = check_launch("koemi_moe_combine(zero)");
        if (st != KOEMI_OK) return st;
        if (pairs > 0) {
            hipLaunchKernelGGL(invert_rows_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0, s, sorted_rows,
                               segment_offsets + num_segments, cnt, pos, pairs, tokens, top_k);
            st = check_launch("koemi_moe_combine(invert)");
            if (st != KOEMI_OK) return st;
        }
    }
    switch (dtype) {
        case KOEMI_F32: return launch_combine_rows<float>(expert_outputs, cnt, pos, pair_weights, combined, tokens, top_k, width, s);
        case KOEMI_F16: return launch_combine_rows<f16>(expert_outputs, cnt, pos, pair_weights, combined, tokens, top_k, width, s);
        default: return launch_combine_rows<bf16>(expert_outputs, cnt, pos, pair_weights, combined, tokens, top_k, width, s);
    }
}


extern "C" int koemi_herm_combine_norm(const void* expert_outputs, const int64_t* sorted_rows,
                                       const int64_t* pair_positions, const int64_t* segment_offsets,
                                       const float* pair_weights, const float* context,
                                       const uint8_t* mask, const float* expert_norm_weight,
                                       const float* next_norm_weight, float* output, void* next_input_bf16,
                                       int64_t pairs, int64_t width, int64_t tokens, int64_t top_k,
                                       int64_t num_segments, float eps, void* workspace, size_t workspace_bytes,
                                       koemi_stream_t stream) {
    if (tokens < 1 || width < 1 || pairs < 0) return fail(KOEMI_ERR_INVALID, "combine norm needs tokens, width >= 1");
    if (top_k < 1 || top_k > 8) return fail(KOEMI_ERR_UNSUPPORTED, "combine norm takes top_k in [1, 8]");
    if (num_segments < 1) return fail(KOEMI_ERR_INVALID, "segment_offsets must have at least two entries");
    if (width % 4 != 0 || width > 4 * kWave * 8)
        return fail(KOEMI_ERR_UNSUPPORTED, "combine norm needs a width that is a multiple of 4 and at most 2048");
    if (!segment_offsets || !context || !expert_norm_weight ||
        (pairs > 0 && (!expert_outputs || (!sorted_rows && !pair_positions))))
        return fail(KOEMI_ERR_INVALID, "combine norm received a null pointer");
    if (!output && !(next_norm_weight && next_input_bf16))
        return fail(KOEMI_ERR_INVALID, "combine norm has no output");
    if ((reinterpret_cast<uintptr_t>(expert_outputs) | reinterpret_cast<uintptr_t>(context) |
         reinterpret_cast<uintptr_t>(output) | reinterpret_cast<uintptr_t>(next_input_bf16)) % 16)
        return fail(KOEMI_ERR_UNSUPPORTED, "combine norm needs 16-byte aligned rows");
    hipStream_t s = as_stream(stream);
    const dim3 grid(grid_for(tokens, kCombineWaves)), block(kWave * kCombineWaves);
    const bf16* y = static_cast<const bf16*>(expert_outputs);
    bf16* o16 = static_cast<bf16*>(next_input_bf16);
    const int H = static_cast<int>(width);
    const bool wide = width > 4 * kWave * 4;
    const int64_t* valid_end = segment_offsets + num_segments;
    auto launch = [&](auto kernel, const int32_t* cnt, const int64_t* pos) {
        hipLaunchKernelGGL(kernel, grid, block, 0, s, y, cnt, pos, valid_end, pair_weights, context, mask,
                           expert_norm_weight, next_norm_weight, output, o16, tokens, top_k, H, eps,
                           static_cast<const bf16*>(nullptr), static_cast<const float*>(nullptr));
        return check_launch("koemi_herm_combine_norm(rows)");
    };
    if (pair_positions != nullptr) {  // the permutation's own map: no inversion
        if (top_k <= 2 && !wide && tokens <= 1024)
            return launch(combine_norm_kernel<2, 4, true, true>, nullptr, pair_positions);
        if (top_k <= 2) return wide ? launch(combine_norm_kernel<2, 8, true>, nullptr, pair_positions)
                                    : launch(combine_norm_kernel<2, 4, true>, nullptr, pair_positions);
        if (top_k <= 4) return wide ? launch(combine_norm_kernel<4, 8, true>, nullptr, pair_positions)
                                    : launch(combine_norm_kernel<4, 4, true>, nullptr, pair_positions);
        return wide ? launch(combine_norm_kernel<8, 8, true>, nullptr, pair_positions)
                    : launch(combine_norm_kernel<8, 4, true>, nullptr, pair_positions);
    }
    const CombineWorkspace ws = combine_workspace(tokens, top_k);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "combine norm workspace too small: need %zu bytes", ws.total);
    char* base = static_cast<char*>(workspace);
    int32_t* cnt = reinterpret_cast<int32_t*>(base + ws.cnt_off);
    int64_t* pos = reinterpret_cast<int64_t*>(base + ws.pos_off);
    int st = KOEMI_OK;
    if (tokens <= kSmallInvertTokens && pairs <= 4096) {
        hipLaunchKernelGGL(invert_rows_small_kernel, dim3(1), dim3(1024), 0, s, sorted_rows,
                           segment_offsets + num_segments, cnt, pos, pairs, tokens, top_k);
        st = check_launch("koemi_herm_combine_norm(invert)");
    } else {
        hipLaunchKernelGGL(zero_i32_kernel, dim3(grid_for(tokens, 256)), dim3(256), 0, s, cnt, tokens);
        st = check_launch("koemi_herm_combine_norm(zero)");
        if (st == KOEMI_OK && pairs > 0) {
            hipLaunchKernelGGL(invert_rows_kernel, dim3(grid_for(pairs, 256)), dim3(256), 0, s, sorted_rows,
                               segment_offsets + num_segments, cnt, pos, pairs, tokens, top_k);
            st = check_launch("koemi_herm_combine_norm(invert)");
        }
    }
    if (st != KOEMI_OK) return st;
    if (top_k <= 2) return wide ? launch(combine_norm_kernel<2, 8, false>, cnt, pos)
                                : launch(combine_norm_kernel<2, 4, false>, cnt, pos);
    if (top_k <= 4) return wide ? launch(combine_norm_kernel<4, 8, false>, cnt, pos)
                                : launch(combine_norm_kernel<4, 4, false>, cnt, pos);
    return wide ? launch(combine_norm_kernel<8, 8, false>, cnt, pos)
                : launch(combine_norm_kernel<8, 4, false>, cnt, pos);
}

extern "C" int koemi_herm_combine_norm_fusion(const void* expert_outputs, const int64_t* pair_positions,
                                              const int64_t* segment_offsets, const float* pair_weights,
                                              const void* fusion_rows, const float* fusion_norm_weight,
                                              const uint8_t* mask, const float* expert_norm_weight,
                                              const float* next_norm_weight, float* output, void* next_input_bf16,
                                              int64_t pairs, int64_t width, int64_t tokens, int64_t top_k,
                                              int64_t num_segments, float eps, koemi_stream_t stream) {
    if (tokens < 1 || width < 1 || pairs < 0) return fail(KOEMI_ERR_INVALID, "combine norm needs tokens, width >= 1");
    if (top_k < 1 || top_k > 8) return fail(KOEMI_ERR_UNSUPPORTED, "combine norm takes top_k in [1, 8]");
    if (num_segments < 1) return fail(KOEMI_ERR_INVALID, "segment_offsets must have at least two entries");
    if (width % 4 != 0 || width > 4 * kWave * 8)
        return fail(KOEMI_ERR_UNSUPPORTED, "combine norm needs a width that is a multiple of 4 and at most 2048");
    if (!segment_offsets || !fusion_rows || !fusion_norm_weight || !expert_norm_weight || !pair_positions ||
        (pairs > 0 && !expert_outputs))
        return fail(KOEMI_ERR_INVALID, "combine norm received a null pointer");
    if (!output && !(next_norm_weight && next_input_bf16))
        return fail(KOEMI_ERR_INVALID, "combine norm has no output");
    if ((reinterpret_cast<uintptr_t>(expert_outputs) | reinterpret_cast<uintptr_t>(fusion_rows) |
         reinterpret_cast<uintptr_t>(fusion_norm_weight) | reinterpret_cast<uintptr_t>(output) |
         reinterpret_cast<uintptr_t>(next_input_bf16)) % 16)
        return fail(KOEMI_ERR_UNSUPPORTED, "combine norm needs 16-byte aligned rows");
    hipStream_t s = as_stream(stream);
    const dim3 grid(grid_for(tokens, kCombineWaves)), block(kWave * kCombineWaves);
    const bf16* y = static_cast<const bf16*>(expert_outputs);
    bf16* o16 = static_cast<bf16*>(next_input_bf16);
    const bf16* fr = static_cast<const bf16*>(fusion_rows);
    const int H = static_cast<int>(width);
    const bool wide = width > 4 * kWave * 4;
    const int64_t* valid_end = segment_offsets + num_segments;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, block, 0, s, y, static_cast<const int32_t*>(nullptr), pair_positions,
                           valid_end, pair_weights, static_cast<const float*>(nullptr), mask, expert_norm_weight,
                           next_norm_weight, output, o16, tokens, top_k, H, eps, fr, fusion_norm_weight);
        return check_launch("koemi_herm_combine_norm_fusion");
    };
    if (top_k <= 2) return wide ? launch(combine_norm_kernel<2, 8, true, false, true>)
                                : launch(combine_norm_kernel<2, 4, true, false, true>);
    if (top_k <= 4) return wide ? launch(combine_norm_kernel<4, 8, true, false, true>)
                                : launch(combine_norm_kernel<4, 4, true, false, true>);
    return wide ? launch(combine_norm_kernel<8, 8, true, false, true>)
                : launch(combine_norm_kernel<8, 4, true, false, true>);
}
