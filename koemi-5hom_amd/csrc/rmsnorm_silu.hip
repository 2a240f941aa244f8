// Fused RMSNorm + SiLU for gfx950.
//
// Reference: src/koemi/cuda_kernels/core/rmsnorm_silu.cu:62-132 (one block per
// row, two global passes over x). Here a row is held in registers by 16, 32 or
// 64 lanes (narrow rows share a wave): each lane loads NV 16-byte vectors (8
// bf16/f16 or 4 fp32 values), the sum of squares is reduced with a xor
// butterfly over the row's lanes, and y = silu(x * inv * w) is produced from
// the same registers, so x is read from HBM exactly once and y written once.
// Rows whose width does not fit that layout use a generic block-per-row path.
#include "common.hpp"

namespace koemi {
namespace {

constexpr int kNormWaves = 4;
// Cache policy of the grouped forward by the size of x: non-temporal loads of
// x above KOEMI_NORM_NT_LOAD_BYTES, else non-temporal stores of y above
// KOEMI_NT_STORE_BYTES (measured at C2, [32768, 512] bf16: 13.4 -> 11.5 us in
// isolation; non-temporal loads and stores together were slower at both C2
// and C3).
#ifndef KOEMI_NORM_NT_LOAD_BYTES
#define KOEMI_NORM_NT_LOAD_BYTES (int64_t(128) << 20)
#endif

__device__ __forceinline__ float silu(float v) {
    // v * sigmoid(v) with the hardware exp2 and reciprocal (1 ulp each).
    const float e = __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float silu_grad(float v) {
    const float e = __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
    const float sg = __builtin_amdgcn_rcpf(1.0f + e);
    return sg * (1.0f + v * (1.0f - sg));
}

template <typename T>
struct Vec16 {
    static constexpr int N = 16 / sizeof(T);
    union {
        uint4 raw;
        T e[N];
    };
};

// NV vectors per lane; row width H must satisfy H % N == 0 and H <= NV*64*N.
// Each wave handles ROWS consecutive rows and issues all of their loads before
// any arithmetic, so ROWS*NV 16-byte loads per lane are in flight at once.
template <typename T, int NV, int ROWS>
__global__ __launch_bounds__(kWave * kNormWaves) void rmsnorm_silu_fwd_wave(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y, float* __restrict__ inv_out,
    int64_t rows, int H, float eps) {
    constexpr int N = Vec16<T>::N;
    const int lane = lane_id();
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kNormWaves + threadIdx.x / kWave) * ROWS;
    if (row0 >= rows) return;
    // Unconditional loads at clamped addresses (no branch around a load), zeroed
    // afterwards where out of range, so all of them are in flight together.
    Vec16<T> xv[ROWS][NV], wv[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int c = (v * kWave + lane) * N;
        wv[v].raw = *reinterpret_cast<const uint4*>(w + min(c, H - N));
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int c = (v * kWave + lane) * N;
            const int64_t rr = min(row0 + r, rows - 1);
            xv[r][v].raw = *reinterpret_cast<const uint4*>(x + rr * H + min(c, H - N));
        }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int c = (v * kWave + lane) * N;
        if (c >= H) wv[v].raw = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (c >= H || row0 + r >= rows) xv[r][v].raw = make_uint4(0, 0, 0, 0);
    }
    float ss[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        ss[r] = 0.0f;
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const float f = to_f32(xv[r][v].e[i]);
                ss[r] = __builtin_fmaf(f, f, ss[r]);
            }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) ss[r] += __shfl_xor(ss[r], off, kWave);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (row0 + r >= rows) break;
        const float inv = rsqrtf(ss[r] / static_cast<float>(H) + eps);
        if (lane == r) inv_out[row0 + r] = inv;
        T* yr = y + (row0 + r) * H;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int c = (v * kWave + lane) * N;
            if (c < H) {
                Vec16<T> o;
#pragma unroll
                for (int i = 0; i < N; ++i)
                    o.e[i] = from_f32<T>(silu(to_f32(xv[r][v].e[i]) * inv * to_f32(wv[v].e[i])));
                *reinterpret_cast<uint4*>(yr + c) = o.raw;
            }
        }
    }
}

// LPR lanes per row, 64 / LPR rows side by side in a wave (lane l serves row
// l / LPR); each lane holds NV 16-byte vectors of its row at columns
// (v * LPR + l % LPR) * N. Narrow rows keep every lane busy this way and the
// sum of squares needs only log2(LPR) butterfly steps for all rows at once.
// STREAM: x is read with non-temporal loads (inputs much larger than the
// 256 MiB Infinity Cache gain nothing from being cached there, and leaving it
// to the output measured 12% faster at [131072, 1024] bf16).
typedef unsigned int u32x4n __attribute__((ext_vector_type(4)));
template <bool STREAM>
__device__ __forceinline__ uint4 load16(const void* p) {
    if constexpr (STREAM) {
        const u32x4n v = __builtin_nontemporal_load(reinterpret_cast<const u32x4n*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *reinterpret_cast<const uint4*>(p);
    }
}

template <typename T, int NV, int LPR, bool STREAM, bool NT_STORE>
__global__ __launch_bounds__(kWave * kNormWaves) void rmsnorm_silu_fwd_group(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y, float* __restrict__ inv_out,
    int64_t rows, int H, float eps) {
    constexpr int N = Vec16<T>::N;
    constexpr int kRowsPerWave = kWave / LPR;
    const int lane = lane_id();
    const int sub = lane % LPR;
    const int64_t wave_row0 = (static_cast<int64_t>(blockIdx.x) * kNormWaves + threadIdx.x / kWave) * kRowsPerWave;
    if (wave_row0 >= rows) return;
    const int64_t row = wave_row0 + lane / LPR;
    const int64_t rr = row < rows ? row : rows - 1;
    // Unconditional loads at clamped addresses, zeroed afterwards where out of range.
    Vec16<T> xv[NV], wv[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int c = (v * LPR + sub) * N;
        wv[v].raw = *reinterpret_cast<const uint4*>(w + min(c, H - N));
        xv[v].raw = load16<STREAM>(x + rr * H + min(c, H - N));
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int c = (v * LPR + sub) * N;
        if (c >= H) {
            wv[v].raw = make_uint4(0, 0, 0, 0);
            xv[v].raw = make_uint4(0, 0, 0, 0);
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float f = to_f32(xv[v].e[i]);
            ss = __builtin_fmaf(f, f, ss);
        }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
    if (row >= rows) return;
    const float inv = rsqrtf(ss / static_cast<float>(H) + eps);
    if (sub == 0) inv_out[row] = inv;
    T* yr = y + row * H;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int c = (v * LPR + sub) * N;
        if (c < H) {
            Vec16<T> o;
#pragma unroll
            for (int i = 0; i < N; ++i) o.e[i] = from_f32<T>(silu(to_f32(xv[v].e[i]) * inv * to_f32(wv[v].e[i])));
            if constexpr (NT_STORE) store16_nt(yr + c, o.raw);
            else *reinterpret_cast<uint4*>(yr + c) = o.raw;
        }
    }
}

// Generic path: one 256-thread block per row, two passes over the row.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_silu_fwd_block(const T* __restrict__ x,
                                                              const T* __restrict__ w,
                                                              T* __restrict__ y,
                                                              float* __restrict__ inv_out,
                                                              int64_t rows, int H, float eps) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const T* xr = x + row * H;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < H; c += 256) {
        const float f = to_f32(xr[c]);
        ss = __builtin_fmaf(f, f, ss);
    }
    ss = wave_sum_xor(ss);
    if (lane_id() == 0) red[threadIdx.x / kWave] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = rsqrtf(ss / static_cast<float>(H) + eps);
    if (threadIdx.x == 0) inv_out[row] = inv;
    for (int c = threadIdx.x; c < H; c += 256)
        y[row * H + c] = from_f32<T>(silu(to_f32(xr[c]) * inv * to_f32(w[c])));
}

// ------------------------------------------------------------------ backward --
// dx = inv * d * w - x * inv^3 / H * sum_c(d_c w_c x_c),  d = g * silu'(x inv w),
// dw = sum_rows d * x * inv. Stage 1 writes one fp32 partial row of dw per
// workgroup; stage 2 sums the partials in a fixed order (deterministic).
constexpr int kBwdBlockRows = 32;    // rows per workgroup in stage 1 (upper bound on partial count)
constexpr int kBwdMaxBlocks = 1024;

inline int64_t bwd_blocks(int64_t rows) {
    int64_t b = (rows + kBwdBlockRows - 1) / kBwdBlockRows;
    if (b > kBwdMaxBlocks) b = kBwdMaxBlocks;
    if (b < 1) b = 1;
    return b;
}

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_silu_bwd_stage1(
    const T* __restrict__ g, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ inv_rms, T* __restrict__ dx, float* __restrict__ partial,
    int64_t rows, int H) {
    __shared__ float red[4];
    __shared__ float total;
    const int64_t blocks = gridDim.x;
    float* part = partial + static_cast<int64_t>(blockIdx.x) * H;
    for (int c = threadIdx.x; c < H; c += 256) part[c] = 0.0f;
    for (int64_t row = blockIdx.x; row < rows; row += blocks) {
        const T* xr = x + row * H;
        const T* gr = g + row * H;
        const float inv = inv_rms[row];
        float dot = 0.0f;
        for (int c = threadIdx.x; c < H; c += 256) {
            const float xf = to_f32(xr[c]), wf = to_f32(w[c]);
            const float d = to_f32(gr[c]) * silu_grad(xf * inv * wf);
            dot = __builtin_fmaf(d * wf, xf, dot);
        }
        dot = wave_sum_xor(dot);
        __syncthreads();
        if (lane_id() == 0) red[threadIdx.x / kWave] = dot;
        __syncthreads();
        if (threadIdx.x == 0) total = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
        const float corr = inv * inv * inv / static_cast<float>(H) * total;
        for (int c = threadIdx.x; c < H; c += 256) {
            const float xf = to_f32(xr[c]), wf = to_f32(w[c]);
            const float nrm = xf * inv;
            const float d = to_f32(gr[c]) * silu_grad(nrm * wf);
            dx[row * H + c] = from_f32<T>(inv * d * wf - xf * corr);
            part[c] += d * nrm;  // this thread is the only writer of part[c]
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_silu_bwd_stage2(const float* __restrict__ partial,
                                                               T* __restrict__ dw, int64_t blocks,
                                                               int H) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= H) return;
    float acc = 0.0f;
    for (int64_t b = 0; b < blocks; ++b) acc += partial[b * H + c];
    dw[c] = from_f32<T>(acc);
}

template <typename T>
int launch_forward(const void* x, const void* w, void* y, float* inv, int64_t rows, int64_t H,
                   float eps, hipStream_t stream) {
    constexpr int N = Vec16<T>::N;
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    T* yp = static_cast<T*>(y);
    const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(w) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(y) % 16 == 0);
    const int Hi = static_cast<int>(H);
    const dim3 wblock(kWave * kNormWaves);
    if (aligned && H % N == 0) {
        const int64_t vecs = H / N;  // vectors per row
#define KOEMI_NORM_LAUNCH(NV, ROWS)                                                                      \
    hipLaunchKernelGGL((rmsnorm_silu_fwd_wave<T, NV, ROWS>), dim3(grid_for(rows, kNormWaves * ROWS)), wblock, 0, \
                       stream, xp, wp, yp, inv, rows, Hi, eps);                                           \
    return check_launch("koemi_rmsnorm_silu_forward")
        const int64_t bytes = rows * H * static_cast<int64_t>(sizeof(T));
        const bool stream_x = bytes > KOEMI_NORM_NT_LOAD_BYTES;
        const bool nt_store = bytes > KOEMI_NT_STORE_BYTES && !stream_x;  // both together measured slower
#define KOEMI_NORM_GROUP(NV, LPR)                                                                        \
    {                                                                                                    \
        const dim3 g(grid_for(rows, kNormWaves * (kWave / LPR)));                                        \
        if (stream_x)                                                                                    \
            hipLaunchKernelGGL((rmsnorm_silu_fwd_group<T, NV, LPR, true, false>), g, wblock, 0, stream, xp, wp, yp, \
                               inv, rows, Hi, eps);                                                      \
        else if (nt_store)                                                                               \
            hipLaunchKernelGGL((rmsnorm_silu_fwd_group<T, NV, LPR, false, true>), g, wblock, 0, stream, xp, wp, yp, \
                               inv, rows, Hi, eps);                                                      \
        else                                                                                             \
            hipLaunchKernelGGL((rmsnorm_silu_fwd_group<T, NV, LPR, false, false>), g, wblock, 0, stream, xp, wp, yp, \
                               inv, rows, Hi, eps);                                                      \
        return check_launch("koemi_rmsnorm_silu_forward");                                              \
    }
        if (vecs <= 16) { KOEMI_NORM_GROUP(1, 16); }
        if (vecs <= 32) { KOEMI_NORM_GROUP(2, 16); }
        if (vecs <= kWave * 1) { KOEMI_NORM_GROUP(4, 16); }
        if (vecs <= kWave * 2) { KOEMI_NORM_GROUP(4, 32); }
        if (vecs <= kWave * 4) { KOEMI_NORM_LAUNCH(4, 1); }
        if (vecs <= kWave * 8) { KOEMI_NORM_LAUNCH(8, 1); }
#undef KOEMI_NORM_LAUNCH
#undef KOEMI_NORM_GROUP
    }
    if (rows > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "rmsnorm_silu: too many rows for the generic path");
    hipLaunchKernelGGL(rmsnorm_silu_fwd_block<T>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, stream, xp, wp, yp, inv, rows, Hi, eps);
    return check_launch("koemi_rmsnorm_silu_forward");
}

template <typename T>
int launch_backward(const void* g, const void* x, const void* w, const float* inv, void* dx,
                    void* dw, int64_t rows, int64_t H, float* partial, hipStream_t stream) {
    const int64_t blocks = bwd_blocks(rows);
    hipLaunchKernelGGL(rmsnorm_silu_bwd_stage1<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<const T*>(g), static_cast<const T*>(x), static_cast<const T*>(w), inv,
                       static_cast<T*>(dx), partial, rows, static_cast<int>(H));
    int st = check_launch("koemi_rmsnorm_silu_backward");
    if (st != KOEMI_OK) return st;
    hipLaunchKernelGGL(rmsnorm_silu_bwd_stage2<T>, dim3(grid_for(H, 256)), dim3(256), 0, stream, partial,
                       static_cast<T*>(dw), blocks, static_cast<int>(H));
    return check_launch("koemi_rmsnorm_silu_backward");
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_rmsnorm_silu_forward(const void* input, const void* weight, void* output,
                                          float* inverse_rms, int64_t rows, int64_t hidden,
                                          double eps, int dtype, koemi_stream_t stream) {
    if (rows < 0 || hidden < 1) return fail(KOEMI_ERR_INVALID, "rmsnorm_silu needs rows >= 0 and a positive hidden dimension");
    if (hidden > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "rmsnorm_silu hidden dimension too large");
    if (!(eps > 0.0)) return fail(KOEMI_ERR_INVALID, "eps must be finite and positive");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "rmsnorm_silu does not support dtype %s", dtype_name(dtype));
    if (rows == 0) return KOEMI_OK;
    if (!input || !weight || !output || !inverse_rms) return fail(KOEMI_ERR_INVALID, "rmsnorm_silu received a null pointer");
    hipStream_t s = as_stream(stream);
    const float e = static_cast<float>(eps);
    switch (dtype) {
        case KOEMI_F32: return launch_forward<float>(input, weight, output, inverse_rms, rows, hidden, e, s);
        case KOEMI_F16: return launch_forward<f16>(input, weight, output, inverse_rms, rows, hidden, e, s);
        default: return launch_forward<bf16>(input, weight, output, inverse_rms, rows, hidden, e, s);
    }
}

extern "C" size_t koemi_rmsnorm_silu_backward_workspace_bytes(int64_t rows, int64_t hidden) {
    if (rows < 0 || hidden < 1) return 0;
    return static_cast<size_t>(bwd_blocks(rows)) * static_cast<size_t>(hidden) * sizeof(float);
}

extern "C" int koemi_rmsnorm_silu_backward(const void* grad_output, const void* input,
                                           const void* weight, const float* inverse_rms,
                                           void* grad_input, void* grad_weight, int64_t rows,
                                           int64_t hidden, int dtype, void* workspace,
                                           size_t workspace_bytes, koemi_stream_t stream) {
    if (rows < 0 || hidden < 1) return fail(KOEMI_ERR_INVALID, "rmsnorm_silu backward needs rows >= 0 and a positive hidden dimension");
    if (hidden > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "rmsnorm_silu hidden dimension too large");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "rmsnorm_silu does not support dtype %s", dtype_name(dtype));
    if (!grad_weight) return fail(KOEMI_ERR_INVALID, "rmsnorm_silu backward received a null pointer");
    if (rows > 0 && (!grad_output || !input || !weight || !inverse_rms || !grad_input))
        return fail(KOEMI_ERR_INVALID, "rmsnorm_silu backward received a null pointer");
    const size_t need = koemi_rmsnorm_silu_backward_workspace_bytes(rows, hidden);
    if (workspace_bytes < need || (need > 0 && !workspace))
        return fail(KOEMI_ERR_INVALID, "rmsnorm_silu backward workspace too small: need %zu bytes", need);
    hipStream_t s = as_stream(stream);
    float* partial = static_cast<float*>(workspace);
    switch (dtype) {
        case KOEMI_F32: return launch_backward<float>(grad_output, input, weight, inverse_rms, grad_input, grad_weight, rows, hidden, partial, s);
        case KOEMI_F16: return launch_backward<f16>(grad_output, input, weight, inverse_rms, grad_input, grad_weight, rows, hidden, partial, s);
        default: return launch_backward<bf16>(grad_output, input, weight, inverse_rms, grad_input, grad_weight, rows, hidden, partial, s);
    }
}
