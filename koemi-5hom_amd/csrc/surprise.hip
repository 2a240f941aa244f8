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

// NCH > 0: each row has at most NCH*256 logits and is held in registers; a wave
// handles ROWS rows. Every load of the wave (valid flags, targets, logits) is
// issued up front at a clamped, in-bounds address and out-of-range values are
// replaced afterwards, so the loads overlap instead of waiting one by one; the
// target logit is taken from the register of the lane that holds it.
// VEC: the rows are read as 16-byte vectors (V % 4 == 0 and 16-byte alignment).
// NCH == 0: generic path (one row per wave) that re-reads the row (same element
// ownership and summation order).
template <typename T, int NCH, int ROWS, bool VEC, bool HAS_BIAS>
__global__ __launch_bounds__(kWave * kRowWaves) void surprise_rows_kernel(
    const float* __restrict__ logits, const T* __restrict__ bias,
    const int64_t* __restrict__ targets, const uint8_t* __restrict__ valid, T* __restrict__ out,
    int64_t rows, int64_t V, float log_vocab) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave) * ROWS;
    if (row0 >= rows) return;
    const int64_t nchunks = (V + 255) / 256;
    float m[ROWS], sum[ROWS], zt[ROWS];
    bool live[ROWS];
    int64_t tgt[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const int64_t rr = min(row0 + r, rows - 1);
        live[r] = valid[rr] != 0;
        tgt[r] = targets[rr];
        m[r] = -__builtin_inff();
        sum[r] = 0.0f;
    }
    if constexpr (NCH > 0) {
        // Bias values of this lane's columns (the same for every row).
        float bv[NCH][4];
#pragma unroll
        for (int k = 0; k < NCH; ++k)
#pragma unroll
            for (int p = 0; p < 4; ++p)
                bv[k][p] = HAS_BIAS ? to_f32(bias[min(static_cast<int64_t>(k) * 256 + lane * 4 + p, V - 1)]) : 0.0f;
        float v[ROWS][NCH][4];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const float* z = logits + min(row0 + r, rows - 1) * V;
#pragma unroll
            for (int k = 0; k < NCH; ++k) {
                const int64_t j0 = static_cast<int64_t>(k) * 256 + lane * 4;
                if constexpr (VEC) {
                    const float4 q = *reinterpret_cast<const float4*>(z + min(j0, V - 4));
                    v[r][k][0] = q.x; v[r][k][1] = q.y; v[r][k][2] = q.z; v[r][k][3] = q.w;
                } else {
#pragma unroll
                    for (int p = 0; p < 4; ++p) v[r][k][p] = z[min(j0 + p, V - 1)];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int k = 0; k < NCH; ++k) {
                const int64_t j0 = static_cast<int64_t>(k) * 256 + lane * 4;
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const bool in = k < nchunks && j0 + p < V;
                    if (HAS_BIAS) v[r][k][p] = v[r][k][p] + bv[k][p];
                    if (!in) v[r][k][p] = -__builtin_inff();
                    m[r] = fmaxf(m[r], v[r][k][p]);
                }
            }
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1)
#pragma unroll
            for (int r = 0; r < ROWS; ++r) m[r] = fmaxf(m[r], __shfl_xor(m[r], off, kWave));
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            // z[target] lives in lane (t/4)%64, chunk t/256, component t%4.
            const int64_t t = tgt[r];
            const int owner = static_cast<int>((t >> 2) & 63);
            float mine = 0.0f;
#pragma unroll
            for (int k = 0; k < NCH; ++k)
#pragma unroll
                for (int p = 0; p < 4; ++p)
                    if ((t >> 8) == k && (t & 3) == p) mine = v[r][k][p];
            zt[r] = __shfl(mine, owner, kWave);
#pragma unroll
            for (int k = 0; k < NCH; ++k) {
                const int64_t j0 = static_cast<int64_t>(k) * 256 + lane * 4;
#pragma unroll
                for (int p = 0; p < 4; ++p)
                    if (j0 + p < V) sum[r] = sum[r] + det_expf(v[r][k][p] - m[r]);
            }
        }
    } else {
        static_assert(ROWS == 1 || NCH > 0, "the generic path handles one row per wave");
        const float* z = logits + row0 * V;
        if (live[0]) {
            for (int64_t k = 0; k < nchunks; ++k) {
                const int64_t j0 = k * 256 + lane * 4;
                for (int p = 0; p < 4; ++p)
                    if (j0 + p < V) m[0] = fmaxf(m[0], z[j0 + p] + load_bias(bias, j0 + p));
            }
        }
        m[0] = wave_max_xor(m[0]);
        if (live[0]) {
            for (int64_t k = 0; k < nchunks; ++k) {
                const int64_t j0 = k * 256 + lane * 4;
                for (int p = 0; p < 4; ++p)
                    if (j0 + p < V) sum[0] = sum[0] + det_expf((z[j0 + p] + load_bias(bias, j0 + p)) - m[0]);
            }
        }
        const int64_t t = tgt[0];
        zt[0] = (live[0] && t >= 0 && t < V) ? z[t] + load_bias(bias, t) : 0.0f;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) sum[r] = sum[r] + __shfl_xor(sum[r], off, kWave);
    // Lane r finishes row r.
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (lane != r || row0 + r >= rows) continue;
        float s = 0.0f;
        if (live[r]) {
            const int64_t t = tgt[r];
            if (t < 0 || t >= V) {
                s = __builtin_nanf("");
            } else {
                const float nll = (det_logf(sum[r]) + m[r]) - zt[r];
                s = 1.0f - det_expf(-nll / log_vocab);
            }
        }
        out[row0 + r] = from_f32<T>(s);
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
// at most 4096 buckets of width 2^shift in LDS and keeps the bucket that holds
// the target rank. The key range shrinks 2048-fold or more per pass, so three
// passes reach a single key (two for the usual spread of scores).
//
// For n <= 1024 * NPT the keys are loaded once into registers (all loads in
// flight together) and every pass runs from registers; larger inputs re-read the
// scores from L2 in each pass.
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

// Scores held in registers: element j of thread tid is index j * kSelThreads + tid.
template <int NPT>
struct RegisterKeys {
    uint32_t key[NPT];
    uint64_t present;  // bit j: index in range and score not NaN
    __device__ void load(const float* __restrict__ s, int64_t n) {
        float v[NPT];
#pragma unroll
        for (int j = 0; j < NPT; ++j) {  // unconditional loads at clamped indices
            const int64_t i = static_cast<int64_t>(j) * kSelThreads + threadIdx.x;
            v[j] = s[i < n ? i : n - 1];
        }
#pragma unroll
        for (int j = 0; j < NPT; ++j)
            if (static_cast<int64_t>(j) * kSelThreads + threadIdx.x >= n) v[j] = __builtin_nanf("");
        present = 0;
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            key[j] = order_key(v[j]);
            if (v[j] == v[j]) present |= (1ull << j);
        }
    }
    template <class F>
    __device__ void visit(F f) const {
#pragma unroll
        for (int j = 0; j < NPT; ++j)
            if ((present >> j) & 1ull) f(key[j]);
    }
    __device__ void write_mask(const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm, int64_t n, float tau) const {
        uint8_t ok[NPT];
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int64_t i = static_cast<int64_t>(j) * kSelThreads + threadIdx.x;
            ok[j] = valid[i < n ? i : n - 1];
        }
#pragma unroll
        for (int j = 0; j < NPT; ++j) {
            const int64_t i = static_cast<int64_t>(j) * kSelThreads + threadIdx.x;
            const bool above = ((present >> j) & 1ull) && key_to_float(key[j]) > tau;
            if (i < n) adm[i] = (ok[j] && above) ? 1 : 0;
        }
    }
};

// Scores re-read from memory in every pass (any n).
struct MemoryKeys {
    const float* s;
    int64_t n;
    __device__ void load(const float* __restrict__ src, int64_t count) {
        s = src;
        n = count;
    }
    template <class F>
    __device__ void visit(F f) const {
        int64_t i = threadIdx.x;
        for (; i + 3 * kSelThreads < n; i += 4 * kSelThreads) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = s[i + u * kSelThreads];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (v[u] == v[u]) f(order_key(v[u]));
        }
        for (; i < n; i += kSelThreads) {
            const float v = s[i];
            if (v == v) f(order_key(v));
        }
    }
    __device__ void write_mask(const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm, int64_t count, float tau) const {
        for (int64_t i = threadIdx.x; i < count; i += kSelThreads) adm[i] = (valid[i] && s[i] > tau) ? 1 : 0;
    }
};

// Key of the element with 0-based rank `target` among the (non-NaN) keys.
template <class Keys>
__device__ uint32_t select_rank(const Keys& keys, uint32_t lo, uint32_t hi, uint32_t target, SelShared& sh) {
    const int tid = threadIdx.x;
    uint32_t below = 0;  // elements with key < lo
    for (int pass = 0; pass < 8 && lo < hi; ++pass) {
        // Bucket width 2^shift with (hi - lo) >> shift < kSelBuckets (12-bit buckets).
        const uint32_t span = hi - lo;
        const int shift = span < kSelBuckets ? 0 : 32 - __builtin_clz(span) - 12;
        for (int i = tid; i < kSelBuckets; i += kSelThreads) sh.hist[i] = 0;
        __syncthreads();
        const uint32_t lo_k = lo, hi_k = hi;
        keys.visit([&](uint32_t k) {
            if (k >= lo_k && k <= hi_k) atomicAdd(&sh.hist[(k - lo_k) >> shift], 1u);
        });
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
        const uint64_t new_lo = static_cast<uint64_t>(lo) + (static_cast<uint64_t>(b) << shift);
        const uint64_t new_hi = new_lo + (uint64_t(1) << shift) - 1;
        lo = static_cast<uint32_t>(new_lo);
        hi = static_cast<uint32_t>(new_hi < hi ? new_hi : hi);
        __syncthreads();
    }
    return lo;
}

template <class Keys>
__global__ __launch_bounds__(kSelThreads) void quantile_admission_kernel(
    const float* __restrict__ s, const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm,
    float* __restrict__ tau_out, int64_t n, int64_t k_lo, int64_t k_hi, float weight) {
    __shared__ SelShared sh;
    Keys keys;
    keys.load(s, n);
    uint32_t counted = 0, kmin = 0xffffffffu, kmax = 0;
    keys.visit([&](uint32_t k) {
        ++counted;
        kmin = min(kmin, k);
        kmax = max(kmax, k);
    });
    counted = block_sum_u32(counted, sh);
    kmin = block_min_u32(kmin, sh);
    kmax = block_max_u32(kmax, sh);
    float tau;
    if (static_cast<int64_t>(counted) != n) {
        tau = __builtin_nanf("");  // a NaN score: torch.quantile propagates NaN
    } else {
        const uint32_t key_lo = select_rank(keys, kmin, kmax, static_cast<uint32_t>(k_lo), sh);
        uint32_t key_hi = key_lo;
        if (k_hi != k_lo) {
            // rank k_hi is key_lo again when more than k_hi elements are <= key_lo,
            // otherwise the smallest key above key_lo.
            uint32_t le = 0, above_min = 0xffffffffu;
            keys.visit([&](uint32_t k) {
                if (k <= key_lo) ++le;
                else above_min = min(above_min, k);
            });
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
    if (threadIdx.x == 0) *tau_out = tau;
    keys.write_mask(valid, adm, n, tau);
}

template <typename T>
int launch_rows(const float* logits, const void* bias, const int64_t* targets, const uint8_t* valid,
                void* out, int64_t rows, int64_t V, float log_vocab, hipStream_t stream) {
    const dim3 block(kWave * kRowWaves);
    const T* b = static_cast<const T*>(bias);
    T* o = static_cast<T*>(out);
    const bool vec = (V & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
#define KOEMI_ROWS_LAUNCH(NCH, ROWS, VEC)                                                                      \
    do {                                                                                                       \
        const dim3 grid(grid_for(rows, kRowWaves * ROWS));                                                     \
        if (b)                                                                                                 \
            hipLaunchKernelGGL((surprise_rows_kernel<T, NCH, ROWS, VEC, true>), grid, block, 0, stream, logits, b, \
                               targets, valid, o, rows, V, log_vocab);                                         \
        else                                                                                                   \
            hipLaunchKernelGGL((surprise_rows_kernel<T, NCH, ROWS, VEC, false>), grid, block, 0, stream, logits, b, \
                               targets, valid, o, rows, V, log_vocab);                                         \
    } while (0)
    if (V <= 256) {
        if (vec) KOEMI_ROWS_LAUNCH(1, 4, true);
        else KOEMI_ROWS_LAUNCH(1, 4, false);
    } else if (V <= 1024) {
        if (vec) KOEMI_ROWS_LAUNCH(4, 1, true);
        else KOEMI_ROWS_LAUNCH(4, 1, false);
    } else {
        KOEMI_ROWS_LAUNCH(0, 1, false);
    }
#undef KOEMI_ROWS_LAUNCH
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
    const hipStream_t s = as_stream(stream);
    if (count <= 16LL * kSelThreads)
        hipLaunchKernelGGL(quantile_admission_kernel<RegisterKeys<16>>, dim3(1), dim3(kSelThreads), 0, s,
                           surprise, valid_mask, admission, threshold_out, count, k_lo, k_hi, weight);
    else if (count <= 32LL * kSelThreads)
        hipLaunchKernelGGL(quantile_admission_kernel<RegisterKeys<32>>, dim3(1), dim3(kSelThreads), 0, s,
                           surprise, valid_mask, admission, threshold_out, count, k_lo, k_hi, weight);
    else if (count <= 64LL * kSelThreads)
        hipLaunchKernelGGL(quantile_admission_kernel<RegisterKeys<64>>, dim3(1), dim3(kSelThreads), 0, s,
                           surprise, valid_mask, admission, threshold_out, count, k_lo, k_hi, weight);
    else
        hipLaunchKernelGGL(quantile_admission_kernel<MemoryKeys>, dim3(1), dim3(kSelThreads), 0, s,
                           surprise, valid_mask, admission, threshold_out, count, k_lo, k_hi, weight);
    return check_launch("koemi_admission_quantile");
}
