// Surprise scoring and salience admission for gfx950.
//
// Reference: src/koemi/cuda_kernels/think/surprise_kernel.cu:84-192 (row kernels
// after an fp32 logits GEMM), model/network.py:677-688 (surprise definition)
// and network.py:349 (admission = valid & surprise > threshold).
//
// One wave owns one row of logits. A lane holds elements j = k*256 + lane*4 + p
// (chunk k, component p) and reads them with one 16-byte load per chunk, so a
// 256-logit row is a single coalesced 1 KiB wave load kept in registers: the row
// is read from HBM once (max, sum-exp and the target logit all come from
// registers). The sum of exponentials is accumulated per lane in (k, p) order and
// then combined by a xor butterfly over the 64 lanes; with the exp/log routines
// of detmath.hpp this fixes every rounding step, which is what lets the
// admission mask be reproduced exactly on the host.
#include "common.hpp"
#include "detmath.hpp"

namespace koemi {
namespace {

using detmath::det_expf;
using detmath::det_logf;

constexpr int kRowWaves = 4;  // waves (rows) per workgroup

template <typename T>
__device__ __forceinline__ float load_bias(const T* bias, int64_t j) {
    return bias ? to_f32(bias[j]) : 0.0f;
}

// NCH > 0: the row has at most NCH*256 logits and is held in registers.
// NCH == 0: generic path that re-reads the row (same ownership and order).
template <typename T, int NCH>
__global__ __launch_bounds__(kWave * kRowWaves) void surprise_rows_kernel(
    const float* __restrict__ logits, const T* __restrict__ bias,
    const int64_t* __restrict__ targets, const uint8_t* __restrict__ valid, T* __restrict__ out,
    int64_t rows, int64_t V, float log_vocab) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
    if (row >= rows) return;
    if (!valid[row]) {
        if (lane == 0) out[row] = from_f32<T>(0.0f);
        return;
    }
    const float* z = logits + row * V;
    const int64_t nchunks = (V + 255) / 256;
    float m = -__builtin_inff();
    float sum = 0.0f;
    if constexpr (NCH > 0) {
        float v[NCH][4];
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int64_t j0 = static_cast<int64_t>(k) * 256 + lane * 4;
            if (k < nchunks && j0 + 3 < V && (V & 3) == 0) {
                const float4 q = *reinterpret_cast<const float4*>(z + j0);
                v[k][0] = q.x; v[k][1] = q.y; v[k][2] = q.z; v[k][3] = q.w;
            } else {
#pragma unroll
                for (int p = 0; p < 4; ++p) v[k][p] = (k < nchunks && j0 + p < V) ? z[j0 + p] : -__builtin_inff();
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                if (bias && j0 + p < V) v[k][p] = v[k][p] + load_bias(bias, j0 + p);
                m = fmaxf(m, v[k][p]);
            }
        }
        m = wave_max_xor(m);
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int64_t j0 = static_cast<int64_t>(k) * 256 + lane * 4;
#pragma unroll
            for (int p = 0; p < 4; ++p)
                if (j0 + p < V) sum = sum + det_expf(v[k][p] - m);
        }
    } else {
        for (int64_t k = 0; k < nchunks; ++k) {
            const int64_t j0 = k * 256 + lane * 4;
            for (int p = 0; p < 4; ++p)
                if (j0 + p < V) m = fmaxf(m, z[j0 + p] + load_bias(bias, j0 + p));
        }
        m = wave_max_xor(m);
        for (int64_t k = 0; k < nchunks; ++k) {
            const int64_t j0 = k * 256 + lane * 4;
            for (int p = 0; p < 4; ++p)
                if (j0 + p < V) sum = sum + det_expf((z[j0 + p] + load_bias(bias, j0 + p)) - m);
        }
    }
    sum = wave_sum_xor(sum);
    if (lane == 0) {
        const int64_t t = targets[row];
        float s;
        if (t < 0 || t >= V) {
            s = __builtin_nanf("");
        } else {
            const float zt = z[t] + load_bias(bias, t);
            const float nll = (det_logf(sum) + m) - zt;
            s = 1.0f - det_expf(-nll / log_vocab);
        }
        out[row] = from_f32<T>(s);
    }
}

// d surprise / d logits (surprise_kernel.cu:136-192):
//   dz_j = g * exp(-nll / lnV) / lnV * (softmax_j - [j == target]).
template <typename T>
__global__ __launch_bounds__(kWave * kRowWaves) void surprise_rows_backward_kernel(
    const float* __restrict__ logits, const T* __restrict__ bias,
    const int64_t* __restrict__ targets, const uint8_t* __restrict__ valid,
    const T* __restrict__ grad, float* __restrict__ grad_logits, int64_t rows, int64_t V,
    float log_vocab) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave;
    if (row >= rows) return;
    const float* z = logits + row * V;
    float* dz = grad_logits + row * V;
    const int64_t t = targets[row];
    if (!valid[row] || t < 0 || t >= V) {
        for (int64_t j = lane; j < V; j += kWave) dz[j] = 0.0f;
        return;
    }
    const int64_t nchunks = (V + 255) / 256;
    float m = -__builtin_inff();
    for (int64_t k = 0; k < nchunks; ++k) {
        const int64_t j0 = k * 256 + lane * 4;
        for (int p = 0; p < 4; ++p)
            if (j0 + p < V) m = fmaxf(m, z[j0 + p] + load_bias(bias, j0 + p));
    }
    m = wave_max_xor(m);
    float sum = 0.0f;
    for (int64_t k = 0; k < nchunks; ++k) {
        const int64_t j0 = k * 256 + lane * 4;
        for (int p = 0; p < 4; ++p)
            if (j0 + p < V) sum = sum + det_expf((z[j0 + p] + load_bias(bias, j0 + p)) - m);
    }
    sum = wave_sum_xor(sum);
    const float zt = z[t] + load_bias(bias, t);
    const float nll = (det_logf(sum) + m) - zt;
    const float g = to_f32(grad[row]);
    const float gnll = g * det_expf(-nll / log_vocab) / log_vocab;
    for (int64_t k = 0; k < nchunks; ++k) {
        const int64_t j0 = k * 256 + lane * 4;
        for (int p = 0; p < 4; ++p) {
            const int64_t j = j0 + p;
            if (j < V) {
                const float prob = det_expf((z[j] + load_bias(bias, j)) - m) / sum;
                dz[j] = gnll * (prob - (j == t ? 1.0f : 0.0f));
            }
        }
    }
}

template <typename T>
__global__ void admission_threshold_kernel(const T* __restrict__ s, const uint8_t* __restrict__ valid,
                                           uint8_t* __restrict__ adm, int64_t n, float thr) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) adm[i] = (valid[i] && to_f32(s[i]) > thr) ? 1 : 0;
}

// ---------------------------------------------------------- quantile select ---
// Exact k-th order statistic of n fp32 scores in one workgroup, by repeated
// bucket refinement over the order-preserving 32-bit key of each float:
// every pass histograms the keys inside the current [lo, hi] key range into
// 4096 equal-width buckets in LDS and keeps the bucket that holds the target
// rank. The key range shrinks at least 4096-fold per pass, so three passes reach
// a single key. Scores stay in L2 between passes (n = 32768 is 128 KiB).
constexpr int kSelThreads = 1024;
constexpr int kSelBuckets = 4096;

__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = detmath::float_to_bits(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return detmath::bits_to_float(u);
}

struct SelShared {
    uint32_t hist[kSelBuckets];
    uint32_t wave_tmp[kSelThreads / kWave];
    uint32_t result[4];
};

__device__ uint32_t block_sum_u32(uint32_t v, SelShared& sh) {
    const int lane = lane_id(), w = threadIdx.x / kWave;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    __syncthreads();
    if (lane == 0) sh.wave_tmp[w] = v;
    __syncthreads();
    uint32_t total = 0;
    for (int i = 0; i < kSelThreads / kWave; ++i) total += sh.wave_tmp[i];
    return total;
}

__device__ uint32_t block_min_u32(uint32_t v, SelShared& sh) {
    const int lane = lane_id(), w = threadIdx.x / kWave;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = min(v, static_cast<uint32_t>(__shfl_xor(v, off, kWave)));
    __syncthreads();
    if (lane == 0) sh.wave_tmp[w] = v;
    __syncthreads();
    uint32_t r = 0xffffffffu;
    for (int i = 0; i < kSelThreads / kWave; ++i) r = min(r, sh.wave_tmp[i]);
    return r;
}

__device__ uint32_t block_max_u32(uint32_t v, SelShared& sh) {
    const int lane = lane_id(), w = threadIdx.x / kWave;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, off, kWave)));
    __syncthreads();
    if (lane == 0) sh.wave_tmp[w] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int i = 0; i < kSelThreads / kWave; ++i) r = max(r, sh.wave_tmp[i]);
    return r;
}

// Key of the element with 0-based rank `target` among the (non-NaN) keys.
__device__ uint32_t select_rank(const float* __restrict__ s, int64_t n, uint32_t lo, uint32_t hi,
                                uint32_t target, SelShared& sh) {
    const int tid = threadIdx.x;
    uint32_t below = 0;  // elements with key < lo
    for (int pass = 0; pass < 8 && lo < hi; ++pass) {
        const uint64_t range = static_cast<uint64_t>(hi) - lo + 1;
        const uint64_t bw = (range + kSelBuckets - 1) / kSelBuckets;
        for (int i = tid; i < kSelBuckets; i += kSelThreads) sh.hist[i] = 0;
        __syncthreads();
        for (int64_t i = tid; i < n; i += kSelThreads) {
            const float f = s[i];
            if (f != f) continue;
            const uint32_t k = order_key(f);
            if (k >= lo && k <= hi) atomicAdd(&sh.hist[(k - lo) / bw], 1u);
        }
        __syncthreads();
        // Exclusive prefix over buckets: each thread owns 4 consecutive buckets.
        constexpr int kPer = kSelBuckets / kSelThreads;
        uint32_t local[kPer];
        uint32_t mine = 0;
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            local[q] = sh.hist[tid * kPer + q];
            mine += local[q];
        }
        // Inclusive scan of `mine` across the block.
        const int lane = lane_id(), w = tid / kWave;
        uint32_t incl = mine;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const uint32_t up = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += up;
        }
        __syncthreads();
        if (lane == kWave - 1) sh.wave_tmp[w] = incl;
        __syncthreads();
        uint32_t wave_base = 0;
        for (int i = 0; i < w; ++i) wave_base += sh.wave_tmp[i];
        uint32_t run = below + wave_base + incl - mine;  // elements before my first bucket
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            if (target >= run && target < run + local[q]) {
                sh.result[0] = static_cast<uint32_t>(tid * kPer + q);
                sh.result[1] = run;
            }
            run += local[q];
        }
        __syncthreads();
        const uint32_t b = sh.result[0];
        below = sh.result[1];
        const uint64_t new_lo = static_cast<uint64_t>(lo) + static_cast<uint64_t>(b) * bw;
        const uint64_t new_hi = new_lo + bw - 1;
        lo = static_cast<uint32_t>(new_lo);
        hi = static_cast<uint32_t>(new_hi < hi ? new_hi : hi);
        __syncthreads();
    }
    return lo;
}

__global__ __launch_bounds__(kSelThreads) void quantile_admission_kernel(
    const float* __restrict__ s, const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm,
    float* __restrict__ tau_out, int64_t n, int64_t k_lo, int64_t k_hi, float weight) {
    __shared__ SelShared sh;
    const int tid = threadIdx.x;
    uint32_t nan_count = 0, kmin = 0xffffffffu, kmax = 0;
    for (int64_t i = tid; i < n; i += kSelThreads) {
        const float f = s[i];
        if (f != f) {
            ++nan_count;
        } else {
            const uint32_t k = order_key(f);
            kmin = min(kmin, k);
            kmax = max(kmax, k);
        }
    }
    nan_count = block_sum_u32(nan_count, sh);
    kmin = block_min_u32(kmin, sh);
    kmax = block_max_u32(kmax, sh);
    float tau;
    if (nan_count > 0) {
        tau = __builtin_nanf("");  // torch.quantile propagates NaN
    } else {
        const uint32_t key_lo = select_rank(s, n, kmin, kmax, static_cast<uint32_t>(k_lo), sh);
        uint32_t key_hi = key_lo;
        if (k_hi != k_lo) {
            // rank k_hi is key_lo again when more than k_hi elements are <= key_lo,
            // otherwise the smallest key above key_lo.
            uint32_t le = 0, above_min = 0xffffffffu;
            for (int64_t i = tid; i < n; i += kSelThreads) {
                const uint32_t k = order_key(s[i]);
                if (k <= key_lo) ++le;
                else above_min = min(above_min, k);
            }
            le = block_sum_u32(le, sh);
            above_min = block_min_u32(above_min, sh);
            key_hi = (le > static_cast<uint32_t>(k_hi)) ? key_lo : above_min;
        }
        const float v_lo = key_to_float(key_lo);
        const float v_hi = key_to_float(key_hi);
        // torch.lerp: small weights interpolate from the start, large from the end.
        tau = weight < 0.5f ? __builtin_fmaf(weight, v_hi - v_lo, v_lo)
                            : __builtin_fmaf(weight - 1.0f, v_hi - v_lo, v_hi);
    }
    if (tid == 0) *tau_out = tau;
    for (int64_t i = tid; i < n; i += kSelThreads) adm[i] = (valid[i] && s[i] > tau) ? 1 : 0;
}

template <typename T>
int launch_rows(const float* logits, const void* bias, const int64_t* targets, const uint8_t* valid,
                void* out, int64_t rows, int64_t V, float log_vocab, hipStream_t stream) {
    const dim3 grid(grid_for(rows, kRowWaves)), block(kWave * kRowWaves);
    const T* b = static_cast<const T*>(bias);
    T* o = static_cast<T*>(out);
    if (V <= 256)
        hipLaunchKernelGGL((surprise_rows_kernel<T, 1>), grid, block, 0, stream, logits, b, targets, valid, o, rows, V, log_vocab);
    else if (V <= 1024)
        hipLaunchKernelGGL((surprise_rows_kernel<T, 4>), grid, block, 0, stream, logits, b, targets, valid, o, rows, V, log_vocab);
    else
        hipLaunchKernelGGL((surprise_rows_kernel<T, 0>), grid, block, 0, stream, logits, b, targets, valid, o, rows, V, log_vocab);
    return check_launch("koemi_surprise_rows_forward");
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_surprise_rows_forward(const float* logits, const void* bias,
                                           const int64_t* target_ids, const uint8_t* valid_mask,
                                           void* surprise, int64_t rows, int64_t vocab,
                                           float log_vocab, int dtype, koemi_stream_t stream) {
    if (rows < 0 || vocab < 1) return fail(KOEMI_ERR_INVALID, "surprise rows need rows >= 0 and vocab >= 1");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "surprise does not support dtype %s", dtype_name(dtype));
    if (rows == 0) return KOEMI_OK;
    if (!logits || !target_ids || !valid_mask || !surprise)
        return fail(KOEMI_ERR_INVALID, "surprise received a null pointer");
    hipStream_t s = as_stream(stream);
    switch (dtype) {
        case KOEMI_F32: return launch_rows<float>(logits, bias, target_ids, valid_mask, surprise, rows, vocab, log_vocab, s);
        case KOEMI_F16: return launch_rows<f16>(logits, bias, target_ids, valid_mask, surprise, rows, vocab, log_vocab, s);
        default: return launch_rows<bf16>(logits, bias, target_ids, valid_mask, surprise, rows, vocab, log_vocab, s);
    }
}

extern "C" int koemi_surprise_rows_backward(const float* logits, const void* bias,
                                            const int64_t* target_ids, const uint8_t* valid_mask,
                                            const void* grad_surprise, float* grad_logits,
                                            int64_t rows, int64_t vocab, float log_vocab,
                                            int dtype, koemi_stream_t stream) {
    if (rows < 0 || vocab < 1) return fail(KOEMI_ERR_INVALID, "surprise rows need rows >= 0 and vocab >= 1");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "surprise does not support dtype %s", dtype_name(dtype));
    if (rows == 0) return KOEMI_OK;
    if (!logits || !target_ids || !valid_mask || !grad_surprise || !grad_logits)
        return fail(KOEMI_ERR_INVALID, "surprise backward received a null pointer");
    hipStream_t s = as_stream(stream);
    const dim3 grid(grid_for(rows, kRowWaves)), block(kWave * kRowWaves);
#define KOEMI_SURPRISE_BWD(T)                                                                       \
    hipLaunchKernelGGL((surprise_rows_backward_kernel<T>), grid, block, 0, s, logits,              \
                       static_cast<const T*>(bias), target_ids, valid_mask,                        \
                       static_cast<const T*>(grad_surprise), grad_logits, rows, vocab, log_vocab)
    switch (dtype) {
        case KOEMI_F32: KOEMI_SURPRISE_BWD(float); break;
        case KOEMI_F16: KOEMI_SURPRISE_BWD(f16); break;
        default: KOEMI_SURPRISE_BWD(bf16); break;
    }
#undef KOEMI_SURPRISE_BWD
    return check_launch("koemi_surprise_rows_backward");
}

extern "C" int koemi_admission_threshold(const void* surprise, const uint8_t* valid_mask,
                                         uint8_t* admission, int64_t count, float threshold,
                                         int dtype, koemi_stream_t stream) {
    if (count < 0) return fail(KOEMI_ERR_INVALID, "admission count must be non-negative");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "admission does not support dtype %s", dtype_name(dtype));
    if (count == 0) return KOEMI_OK;
    if (!surprise || !valid_mask || !admission) return fail(KOEMI_ERR_INVALID, "admission received a null pointer");
    hipStream_t s = as_stream(stream);
    const dim3 grid(grid_for(count, 256)), block(256);
    switch (dtype) {
        case KOEMI_F32: hipLaunchKernelGGL(admission_threshold_kernel<float>, grid, block, 0, s, static_cast<const float*>(surprise), valid_mask, admission, count, threshold); break;
        case KOEMI_F16: hipLaunchKernelGGL(admission_threshold_kernel<f16>, grid, block, 0, s, static_cast<const f16*>(surprise), valid_mask, admission, count, threshold); break;
        default: hipLaunchKernelGGL(admission_threshold_kernel<bf16>, grid, block, 0, s, static_cast<const bf16*>(surprise), valid_mask, admission, count, threshold); break;
    }
    return check_launch("koemi_admission_threshold");
}

extern "C" size_t koemi_admission_quantile_workspace_bytes(int64_t count) {
    (void)count;
    return 0;
}

extern "C" int koemi_admission_quantile(const float* surprise, const uint8_t* valid_mask,
                                        uint8_t* admission, float* threshold_out, int64_t count,
                                        float quantile, void* workspace, size_t workspace_bytes,
                                        koemi_stream_t stream) {
    (void)workspace;
    (void)workspace_bytes;
    if (count < 1) return fail(KOEMI_ERR_INVALID, "quantile admission needs at least one score");
    if (count > 0xffffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "quantile admission supports at most 2^32-1 scores");
    if (!(quantile >= 0.0f && quantile <= 1.0f)) return fail(KOEMI_ERR_INVALID, "quantile must lie in [0, 1]");
    if (!surprise || !valid_mask || !admission || !threshold_out)
        return fail(KOEMI_ERR_INVALID, "quantile admission received a null pointer");
    // Rank arithmetic of torch.quantile: rank = q * (n - 1) in float32.
    const float rank = quantile * static_cast<float>(count - 1);
    const int64_t k_lo = static_cast<int64_t>(rank);
    const int64_t k_hi = static_cast<int64_t>(__builtin_ceilf(rank));
    const float weight = rank - static_cast<float>(k_lo);
    hipLaunchKernelGGL(quantile_admission_kernel, dim3(1), dim3(kSelThreads), 0, as_stream(stream),
                       surprise, valid_mask, admission, threshold_out, count, k_lo, k_hi, weight);
    return check_launch("koemi_admission_quantile");
}
