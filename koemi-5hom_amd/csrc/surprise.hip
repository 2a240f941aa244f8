// Surprise scoring and salience admission for gfx950.
//
// Reference: src/koemi/cuda_kernels/think/surprise_kernel.cu:84-192 (row kernels
// after an fp32 logits GEMM), model/network.py:677-688 (surprise definition)
// and network.py:349 (admission = valid & surprise > threshold).
//
// Rows of up to 256 logits take a quarter wave each (16 lanes, four rows per
// wave side by side); longer rows take a whole wave, a lane holding elements
// j = k*256 + lane*4 + p (chunk k, component p). Either way a row is read from
// HBM once with 16-byte loads and kept in registers (max, sum-exp and the
// target logit all come from registers). The sum of exponentials is
// accumulated per lane in a fixed element order and then combined by a xor
// butterfly over the row's lanes; with the exp/log routines of detmath.hpp this
// fixes every rounding step, which is what lets the admission mask be
// reproduced exactly on the host.
#include "common.hpp"
#include "detmath.hpp"

#include <mutex>
#include <type_traits>

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
                    if (j0 + p < V) sum[r] = sum[r] + detmath::det_expf_nonpos(v[r][k][p] - m[r]);
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
                    if (j0 + p < V) sum[0] = sum[0] + detmath::det_expf_nonpos((z[j0 + p] + load_bias(bias, j0 + p)) - m[0]);
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

// V <= 256: a quarter wave (16 lanes) per row, four rows per wave processed
// side by side. Lane sub of a row holds elements j = u*64 + sub*4 + p (u < 4,
// p < 4), read as four 16-byte loads (for each u the 16 lanes of a row cover
// 256 contiguous bytes). The exponentials are summed per lane in (u, p) order,
// then by a xor butterfly over the 16 lanes (offsets 8, 4, 2, 1); lane 0 of
// each quarter finishes its row. Every load is issued up front at a clamped
// in-bounds address. FULL: V == 256 (no element is past the end of its row).
// SHIFT (the HERM block's surprise of every position from the state before
// it): rows are (b, pos) of a [batch, length] window; row (b, pos) scores the
// logits of row (b, pos - 1), and for pos == 0 row b of `first` (the carried
// state's logits). `admission` (null: none) receives valid && s > threshold.
// LAYERED (a decode step's surprise of every layer at once): rows are
// (layer, b) of [layers, layer_rows]; row (l, b) takes the targets and
// validity of b and the content bias of layer l (layer_bias.p[l]).
constexpr int kMaxLayers = 32;
template <typename T>
struct LayerBias {
    const T* p[kMaxLayers];
};

template <typename T, bool VEC, bool HAS_BIAS, bool FULL, bool SHIFT = false, bool LAYERED = false>
__global__ __launch_bounds__(kWave * kRowWaves) void surprise_rows16_kernel(
    const float* __restrict__ logits, const T* __restrict__ bias,
    const int64_t* __restrict__ targets, const uint8_t* __restrict__ valid, T* __restrict__ out,
    int64_t rows, int64_t v_runtime, float log_vocab, const float* __restrict__ first = nullptr,
    int64_t length = 1, uint8_t* __restrict__ admission = nullptr, float threshold = 0.0f,
    LayerBias<T> layer_bias = {}, int64_t layer_rows = 1) {
#pragma clang fp contract(off)
    const int64_t V = FULL ? 256 : v_runtime;
    const int lane = lane_id();
    const int sub = lane & 15;
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * kRowWaves + threadIdx.x / kWave) * 4 + (lane >> 4);
    if ((row & ~int64_t(3)) >= rows) return;  // whole wave past the end
    const int64_t rr = row < rows ? row : rows - 1;
    const int64_t tr = LAYERED ? rr % layer_rows : rr;  // the row of targets and valid
    if constexpr (LAYERED) bias = layer_bias.p[rr / layer_rows];
    const bool live = valid[tr] != 0;
    const int64_t t = targets[tr];
    const float* z = logits + rr * V;
    if constexpr (SHIFT) {
        const int64_t pos = rr % length;
        z = pos == 0 ? first + (rr / length) * V : logits + (rr - 1) * V;
    }
    float v[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t j0 = u * 64 + sub * 4;
        if constexpr (VEC) {
            const float4 q = *reinterpret_cast<const float4*>(z + min(j0, V - 4));
            v[u][0] = q.x; v[u][1] = q.y; v[u][2] = q.z; v[u][3] = q.w;
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) v[u][p] = z[min(j0 + p, V - 1)];
        }
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t j0 = u * 64 + sub * 4;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            if (HAS_BIAS) v[u][p] = v[u][p] + to_f32(bias[min(j0 + p, V - 1)]);
            if (!FULL && j0 + p >= V) v[u][p] = -__builtin_inff();
            m = fmaxf(m, v[u][p]);
        }
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    // z[target] lives in lane (t % 64) / 4 of the quarter, slot (t / 64, t % 4).
    float mine = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int p = 0; p < 4; ++p)
            if ((t >> 6) == u && (t & 3) == p) mine = v[u][p];
    const float zt = __shfl(mine, (lane & ~15) | static_cast<int>((t >> 2) & 15), kWave);
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t j0 = u * 64 + sub * 4;
#pragma unroll
        for (int p = 0; p < 4; ++p)
            if (FULL || j0 + p < V) sum = sum + detmath::det_expf_nonpos(v[u][p] - m);
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off, kWave);
    if (sub != 0 || row >= rows) return;
    float s = 0.0f;
    if (live) {
        if (t < 0 || t >= V) {
            s = __builtin_nanf("");
        } else {
            const float nll = (det_logf(sum) + m) - zt;
            s = 1.0f - det_expf(-nll / log_vocab);
        }
    }
    out[row] = from_f32<T>(s);
    if (admission != nullptr) admission[row] = (live && to_f32(from_f32<T>(s)) > threshold) ? 1 : 0;
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
            if (j0 + p < V) sum = sum + detmath::det_expf_nonpos((z[j0 + p] + load_bias(bias, j0 + p)) - m);
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
                const float prob = detmath::det_expf_nonpos((z[j] + load_bias(bias, j)) - m) / sum;
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
// Exact order statistics of n fp32 scores in one workgroup, over the
// order-preserving 32-bit key of each float. One pass histograms all keys
// into at most 4096 buckets of width 2^shift spanning [min, max] (LDS atomics)
// and finds, by a prefix over the buckets, the buckets holding ranks k_lo and
// k_hi. When those buckets are small (the usual case: a few dozen scores) their
// keys are gathered into LDS and each candidate counts the smaller and equal
// candidates, which names the key of each rank exactly. Crowded buckets (many
// ties, or a few extreme outliers stretching the range) fall back to repeated
// refinement: each further pass histograms the keys inside the current bucket,
// shrinking the key range 2048-fold or more.
//
// For n <= 1024 * 32 the scores and valid flags are loaded once into
// registers (all loads in flight together), four consecutive elements per
// thread and group so that the mask is written four bytes at a time; larger
// inputs re-read the scores from L2 in each pass.
constexpr int kSelThreads = 1024;
constexpr int kSelBuckets = 4096;
constexpr int kSelList = 512;  // candidates gathered per rank

__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = detmath::float_to_bits(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return detmath::bits_to_float(u);
}

struct SelShared {
    uint32_t hist[kSelBuckets + kWave];  // one spill slot per lane for keys outside the range
    uint32_t list[2][kSelList];
    uint32_t wave_tmp[3][kSelThreads / kWave];
    uint32_t result[8];
};

// Sum, min and max over the workgroup in one exchange.
template <int THREADS = kSelThreads>
__device__ void block_count_min_max(uint32_t& cnt, uint32_t& kmin, uint32_t& kmax, SelShared& sh) {
    const int lane = lane_id(), w = threadIdx.x / kWave;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        cnt += __shfl_xor(cnt, off, kWave);
        kmin = min(kmin, static_cast<uint32_t>(__shfl_xor(kmin, off, kWave)));
        kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(kmax, off, kWave)));
    }
    if (lane == 0) {
        sh.wave_tmp[0][w] = cnt;
        sh.wave_tmp[1][w] = kmin;
        sh.wave_tmp[2][w] = kmax;
    }
    __syncthreads();
    cnt = 0;
    kmin = 0xffffffffu;
    kmax = 0;
#pragma unroll
    for (int i = 0; i < THREADS / kWave; ++i) {
        cnt += sh.wave_tmp[0][i];
        kmin = min(kmin, sh.wave_tmp[1][i]);
        kmax = max(kmax, sh.wave_tmp[2][i]);
    }
    __syncthreads();
}

// Scores held in registers: group g of thread tid holds elements
// 4 * (g * kSelThreads + tid) + c, c < 4.
template <int NPT, bool VEC>
struct RegisterKeys {
    static_assert(NPT % 4 == 0 && NPT <= 32, "four elements per group; 128 VGPRs at 1024 threads");
    static constexpr int kGroups = NPT / 4;
    uint32_t key[NPT];
    uint64_t present;  // bit j: index in range and score not NaN
    uint64_t ok;       // bit j: valid flag
    __device__ static int64_t index(int g, int c) {
        return (static_cast<int64_t>(g) * kSelThreads + threadIdx.x) * 4 + c;
    }
    __device__ void load(const float* __restrict__ s, const uint8_t* __restrict__ valid, int64_t n) {
        float v[NPT];
        uint32_t vw[kGroups];
        // Unconditional loads at clamped indices; VEC: n % 4 == 0, the scores
        // are 16-byte and the flags 4-byte aligned, so each group is one
        // 16-byte and one 4-byte load.
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            if constexpr (VEC) {
                const int64_t i = index(g, 0);
                const int64_t ic = i < n ? i : n - 4;
                const float4 f = *reinterpret_cast<const float4*>(s + ic);
                v[g * 4 + 0] = f.x;
                v[g * 4 + 1] = f.y;
                v[g * 4 + 2] = f.z;
                v[g * 4 + 3] = f.w;
                vw[g] = *reinterpret_cast<const uint32_t*>(valid + ic);
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int64_t i = index(g, c);
                    v[g * 4 + c] = s[i < n ? i : n - 1];
                }
                uint32_t w = 0;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int64_t i = index(g, c);
                    w |= static_cast<uint32_t>(valid[i < n ? i : n - 1]) << (8 * c);
                }
                vw[g] = w;
            }
        }
        present = 0;
        ok = 0;
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int j = g * 4 + c;
                key[j] = order_key(v[j]);
                if (index(g, c) < n && v[j] == v[j]) present |= (1ull << j);
                if ((vw[g] >> (8 * c)) & 0xffu) ok |= (1ull << j);
            }
    }
    template <class F>
    __device__ void visit(F f) const {
#pragma unroll
        for (int j = 0; j < NPT; ++j)
            if ((present >> j) & 1ull) f(key[j]);
    }
    // Every slot, with its presence flag (no branch per element).
    template <class F>
    __device__ void visit_all(F f) const {
#pragma unroll
        for (int j = 0; j < NPT; ++j) f(key[j], ((present >> j) & 1ull) != 0);
    }
    __device__ void write_mask(uint8_t* __restrict__ adm, int64_t n, float tau) const {
#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            uint32_t w = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int j = g * 4 + c;
                const bool on = ((ok >> j) & 1ull) && ((present >> j) & 1ull) && key_to_float(key[j]) > tau;
                w |= static_cast<uint32_t>(on) << (8 * c);
            }
            const int64_t i0 = index(g, 0);
            if constexpr (VEC) {
                if (i0 < n) *reinterpret_cast<uint32_t*>(adm + i0) = w;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (i0 + c < n) adm[i0 + c] = static_cast<uint8_t>((w >> (8 * c)) & 0xffu);
            }
        }
    }
};

// Scores re-read from memory in every pass (any n).
template <int THREADS>
struct MemoryKeys {
    const float* s;
    const uint8_t* valid;
    int64_t n;
    __device__ void load(const float* __restrict__ src, const uint8_t* __restrict__ flags, int64_t count) {
        s = src;
        valid = flags;
        n = count;
    }
    template <class F>
    __device__ void visit(F f) const {
        int64_t i = threadIdx.x;
        for (; i + 3 * THREADS < n; i += 4 * THREADS) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = s[i + u * THREADS];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (v[u] == v[u]) f(order_key(v[u]));
        }
        for (; i < n; i += THREADS) {
            const float v = s[i];
            if (v == v) f(order_key(v));
        }
    }
    template <class F>
    __device__ void visit_all(F f) const {
        visit([&](uint32_t k) { f(k, true); });
    }
    __device__ void write_mask(uint8_t* __restrict__ adm, int64_t count, float tau) const {
        for (int64_t i = threadIdx.x; i < count; i += THREADS) adm[i] = (valid[i] && s[i] > tau) ? 1 : 0;
    }
};

// Histograms the keys in [lo, hi] into kSelBuckets buckets of width 2^shift and
// finds the bucket holding each of the ranks t0 <= t1 (ranks count from the
// start of the range, after `below` smaller keys). Results in sh.result:
// [0] bucket of t0, [1] keys before it, [2] its size, [3..5] the same for t1.
template <class Keys, int THREADS = kSelThreads, int BUCKETS = kSelBuckets>
__device__ void bucket_pass(const Keys& keys, uint32_t lo, uint32_t hi, int shift, uint32_t below, uint32_t t0,
                            uint32_t t1, SelShared& sh) {
    static_assert(BUCKETS <= kSelBuckets && BUCKETS % THREADS == 0, "bucket layout");
    const int tid = threadIdx.x;
    for (int i = tid; i < BUCKETS + kWave; i += THREADS) sh.hist[i] = 0;
    __syncthreads();
    const uint32_t spill = BUCKETS + lane_id();
    keys.visit_all([&](uint32_t k, bool present) {
        const bool in = present && k >= lo && k <= hi;
        atomicAdd(&sh.hist[in ? (k - lo) >> shift : spill], 1u);
    });
    __syncthreads();
    // Exclusive prefix over buckets: each thread owns kPer consecutive buckets.
    constexpr int kPer = BUCKETS / THREADS;
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
    if (lane == kWave - 1) sh.wave_tmp[0][w] = incl;
    __syncthreads();
    uint32_t wave_base = 0;
    for (int i = 0; i < w; ++i) wave_base += sh.wave_tmp[0][i];
    uint32_t run = below + wave_base + incl - mine;  // keys before my first bucket
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        if (t0 >= run && t0 < run + local[q]) {
            sh.result[0] = static_cast<uint32_t>(tid * kPer + q);
            sh.result[1] = run;
            sh.result[2] = local[q];
        }
        if (t1 >= run && t1 < run + local[q]) {
            sh.result[3] = static_cast<uint32_t>(tid * kPer + q);
            sh.result[4] = run;
            sh.result[5] = local[q];
        }
        run += local[q];
    }
    __syncthreads();
}

// Key of the element with 0-based rank `target` among the (non-NaN) keys, by
// repeated bucket refinement.
template <class Keys, int THREADS = kSelThreads>
__device__ uint32_t select_rank(const Keys& keys, uint32_t lo, uint32_t hi, uint32_t target, SelShared& sh) {
    uint32_t below = 0;  // keys < lo
    for (int pass = 0; pass < 8 && lo < hi; ++pass) {
        const uint32_t span = hi - lo;
        const int shift = span < kSelBuckets ? 0 : 32 - __builtin_clz(span) - 12;
        bucket_pass<Keys, THREADS>(keys, lo, hi, shift, below, target, target, sh);
        const uint32_t b = sh.result[0];
        below = sh.result[1];
        __syncthreads();
        const uint64_t new_lo = static_cast<uint64_t>(lo) + (static_cast<uint64_t>(b) << shift);
        const uint64_t new_hi = new_lo + (uint64_t(1) << shift) - 1;
        lo = static_cast<uint32_t>(new_lo);
        hi = static_cast<uint32_t>(new_hi < hi ? new_hi : hi);
    }
    return lo;
}

// Keys of ranks t0 and t1 = t0 or t0 + 1 among the keys in [kmin, kmax].
template <class Keys, int BUCKET_BITS = 12, int THREADS = kSelThreads>
__device__ void select_two_ranks(const Keys& keys, uint32_t kmin, uint32_t kmax, uint32_t t0, uint32_t t1,
                                 SelShared& sh, uint32_t& key0, uint32_t& key1) {
    constexpr int kBuckets = 1 << BUCKET_BITS;
    const int tid = threadIdx.x;
    const uint32_t span = kmax - kmin;
    const int shift = span < kBuckets ? 0 : 32 - __builtin_clz(span) - BUCKET_BITS;
    bucket_pass<Keys, THREADS, kBuckets>(keys, kmin, kmax, shift, 0, t0, t1, sh);
    const uint32_t b0 = sh.result[0], below0 = sh.result[1], n0 = sh.result[2];
    const uint32_t b1 = sh.result[3], below1 = sh.result[4], n1 = sh.result[5];
    __syncthreads();
    if (n0 > kSelList || n1 > kSelList) {  // crowded bucket: refine
        key0 = select_rank<Keys, THREADS>(keys, kmin, kmax, t0, sh);
        key1 = (t1 == t0) ? key0 : select_rank<Keys, THREADS>(keys, kmin, kmax, t1, sh);
        return;
    }
    // Gather the candidates of both buckets (list 1 only when they differ).
    if (tid < 2) sh.result[6 + tid] = 0;
    __syncthreads();
    const uint32_t lo = kmin;
    keys.visit([&](uint32_t k) {
        const uint32_t b = (k - lo) >> shift;
        if (b == b0) sh.list[0][atomicAdd(&sh.result[6], 1u)] = k;
        else if (b == b1) sh.list[1][atomicAdd(&sh.result[7], 1u)] = k;
    });
    __syncthreads();
    // The first half of the threads ranks list 0 for t0, the second half the
    // list of t1 (one entry per thread at 1024 threads).
    constexpr int kHalf = THREADS / 2;
    const int half = tid / kHalf;
    const uint32_t* list = (half == 1 && b1 != b0) ? sh.list[1] : sh.list[0];
    const uint32_t m = (half == 1 && b1 != b0) ? n1 : n0;
    const uint32_t r = half == 0 ? t0 - below0 : t1 - below1;
    for (uint32_t idx = tid % kHalf; idx < m; idx += kHalf) {
        const uint32_t x = list[idx];
        uint32_t less = 0, equal = 0;
        for (uint32_t j = 0; j < m; ++j) {
            const uint32_t y = list[j];
            less += y < x;
            equal += y == x;
        }
        if (less <= r && r < less + equal) sh.result[half] = x;  // equal keys write the same value
    }
    __syncthreads();
    key0 = sh.result[0];
    key1 = sh.result[1];
    __syncthreads();
}

template <class Keys>
__global__ __launch_bounds__(kSelThreads) void quantile_admission_kernel(
    const float* __restrict__ s, const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm,
    float* __restrict__ tau_out, int64_t n, int64_t k_lo, int64_t k_hi, float weight) {
    __shared__ SelShared sh;
    Keys keys;
    keys.load(s, valid, n);
    uint32_t counted = 0, kmin = 0xffffffffu, kmax = 0;
    keys.visit([&](uint32_t k) {
        ++counted;
        kmin = min(kmin, k);
        kmax = max(kmax, k);
    });
    block_count_min_max(counted, kmin, kmax, sh);
    float tau;
    if (static_cast<int64_t>(counted) != n) {
        tau = __builtin_nanf("");  // a NaN score: torch.quantile propagates NaN
    } else {
        uint32_t key_lo, key_hi;
        select_two_ranks(keys, kmin, kmax, static_cast<uint32_t>(k_lo), static_cast<uint32_t>(k_hi), sh, key_lo,
                         key_hi);
        const float v_lo = key_to_float(key_lo);
        const float v_hi = key_to_float(key_hi);
        // torch.lerp: small weights interpolate from the start, large from the end.
        tau = weight < 0.5f ? __builtin_fmaf(weight, v_hi - v_lo, v_lo)
                            : __builtin_fmaf(weight - 1.0f, v_hi - v_lo, v_hi);
    }
    if (threadIdx.x == 0) *tau_out = tau;
    keys.write_mask(adm, n, tau);
}

// ----------------------------------------------- two-kernel quantile select ---
// For larger n the per-element work is spread over many workgroups:
//
//   partition (grid, 4 scores per thread): every workgroup reads the same
//     strided sample of 1024 scores and, from its bucket histogram, the same
//     two pivot keys p_lo <= p_hi bracketing sample ranks a few standard
//     deviations either side of the target ranks. Each workgroup then splits
//     its own scores into below p_lo (mask 0), above p_hi (mask = valid) and
//     candidates, writes the decided mask bytes, and records its counts and
//     its candidates (key; index in the workgroup with the valid flag in bit
//     31) in its own workspace slot (no atomics, so the workspace needs no
//     clearing).
//   finish (one workgroup): every thread loads the records and its share of
//     every slot at once (one memory round trip), checks that the target
//     ranks lie among the candidates, selects their keys exactly from the
//     candidates gathered in LDS, forms tau, checks p_lo <= tau <= p_hi (which
//     makes every decided mask byte correct) and writes the candidates' mask
//     bytes. If a check fails (a NaN score, a sample far off the data, too
//     many candidates) it falls back to the exact single-workgroup select over
//     all scores and rewrites the whole mask.
//
// Both kernels run THREADS threads per workgroup: 256 up to 32768 scores (a
// workgroup of 4 waves finds room on a CU beside other kernels' workgroups,
// so the select can overlap independent work on another stream), 1024 above.
// A workgroup partitions 4 * THREADS scores and keeps up to THREADS
// candidates; the finish loads one slot entry per thread and workgroup.
constexpr int kPartPerThread = 4;
constexpr int kPartMaxGroups = 32;
constexpr int kSampleSize = 1024;
static_assert(static_cast<int64_t>(kSampleSize) * kPartMaxGroups * 1024 * kPartPerThread <= (int64_t(1) << 32),
              "32-bit sample index arithmetic");
constexpr int kSampleBuckets = 1024;
constexpr int kFinishCand = 8192;                            // candidates gathered in LDS
constexpr int kRecordWords = 8;  // per workgroup: below, candidates, NaNs, candidate min / max key
constexpr int64_t kPartitionMin = 8192;                      // smaller inputs: one workgroup
#ifndef KOEMI_PART_SMALL_MAX
#define KOEMI_PART_SMALL_MAX (int64_t(kPartMaxGroups) * 256 * kPartPerThread)
#endif
constexpr int64_t kPartSmallMax = KOEMI_PART_SMALL_MAX;   // 256-thread path
constexpr int64_t kPartMax = int64_t(kPartMaxGroups) * 1024 * kPartPerThread;       // 1024-thread path

inline int part_threads(int64_t n) { return n <= kPartSmallMax ? 256 : 1024; }

struct PartWorkspace {
    int threads, groups;
    size_t header_off, record_off, key_off, index_off, total;
};
inline PartWorkspace part_workspace(int64_t n) {
    PartWorkspace w;
    w.threads = part_threads(n);
    const int64_t scores = int64_t(w.threads) * kPartPerThread;
    w.groups = static_cast<int>((n + scores - 1) / scores);
    const size_t slots = static_cast<size_t>(w.groups) * w.threads * sizeof(uint32_t);
    w.header_off = 0;
    w.record_off = 256;
    w.key_off = w.record_off + ((static_cast<size_t>(w.groups) * kRecordWords * sizeof(uint32_t) + 255) & ~size_t(255));
    w.index_off = w.key_off + ((slots + 255) & ~size_t(255));
    w.total = w.index_off + ((slots + 255) & ~size_t(255));
    return w;
}

// The sample: 256 runs of 4 consecutive scores, run b starting at
// floor(b * n / 256) rounded down to a multiple of 4 (so a run is one 16-byte
// line segment and the sample touches 256 cache lines, not 1024); sample
// element i = 4 b + c is held by thread tid with i = tid + j * THREADS.
// n > 1024 and b * n < 2^32 on the partitioned path, so 32-bit arithmetic is
// exact and every run lies inside the scores.
template <int THREADS>
struct SampleKeys {
    static constexpr int kPer = kSampleSize / THREADS;
    uint32_t key[kPer];
    uint32_t present;  // bit j: key[j] is not NaN
    __device__ void load(const float* __restrict__ s, int64_t n) {
        float v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const uint32_t i = static_cast<uint32_t>(threadIdx.x + j * THREADS);
            const uint32_t run = ((i >> 2) * static_cast<uint32_t>(n) / (kSampleSize / 4)) & ~3u;
            v[j] = s[run + (i & 3u)];
        }
        present = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            key[j] = order_key(v[j]);
            present |= (v[j] == v[j] ? 1u : 0u) << j;
        }
    }
    template <class F>
    __device__ void visit(F f) const {
#pragma unroll
        for (int j = 0; j < kPer; ++j)
            if ((present >> j) & 1u) f(key[j]);
    }
    template <class F>
    __device__ void visit_all(F f) const {
#pragma unroll
        for (int j = 0; j < kPer; ++j) f(key[j], ((present >> j) & 1u) != 0);
    }
};

template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void quantile_partition_kernel(
    const float* __restrict__ s, const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm, int64_t n,
    int64_t k_lo, int64_t k_hi, uint32_t* __restrict__ header, uint32_t* __restrict__ records,
    uint32_t* __restrict__ cand_key, uint32_t* __restrict__ cand_index) {
    __shared__ SelShared sh;
    constexpr int kScores = THREADS * kPartPerThread;  // per workgroup
    constexpr int kCand = THREADS;                      // candidate slots per workgroup
    const int tid = threadIdx.x;
    // Own scores and the sample are loaded together.
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScores + static_cast<int64_t>(tid) * kPartPerThread;
    float v[kPartPerThread];
    uint32_t vw = 0;
    if constexpr (VEC) {
        const int64_t ic = base < n ? base : n - kPartPerThread;
        const float4 f = *reinterpret_cast<const float4*>(s + ic);
        v[0] = f.x;
        v[1] = f.y;
        v[2] = f.z;
        v[3] = f.w;
        vw = *reinterpret_cast<const uint32_t*>(valid + ic);
    } else {
#pragma unroll
        for (int c = 0; c < kPartPerThread; ++c) {
            const int64_t i = base + c < n ? base + c : n - 1;
            v[c] = s[i];
            vw |= static_cast<uint32_t>(valid[i]) << (8 * c);
        }
    }
    SampleKeys<THREADS> sample;
    sample.load(s, n);

    // Pivots from the sample (identical in every workgroup).
    uint32_t m = 0, smin = 0xffffffffu, smax = 0u;
    sample.visit([&](uint32_t k) {
        ++m;
        smin = min(smin, k);
        smax = max(smax, k);
    });
    block_count_min_max<THREADS>(m, smin, smax, sh);
    uint32_t p_lo = 0, p_hi = 0xffffffffu;
    if (m > 0) {
        const float frac0 = static_cast<float>(k_lo) / static_cast<float>(n);
        const float frac1 = static_cast<float>(k_hi) / static_cast<float>(n);
        const float sd = __builtin_sqrtf(static_cast<float>(m) * frac0 * (1.0f - frac0));
        const float margin = 4.0f * sd + 4.0f;
        const float r0f = frac0 * static_cast<float>(m) - margin;
        const float r1f = frac1 * static_cast<float>(m) + margin;
        const uint32_t r0 = r0f <= 0.0f ? 0u : min(static_cast<uint32_t>(r0f), m - 1);
        const uint32_t r1 = r1f >= static_cast<float>(m - 1) ? m - 1 : static_cast<uint32_t>(r1f);
        const uint32_t span = smax - smin;
        const int shift = span < kSampleBuckets ? 0 : 32 - __builtin_clz(span) - 10;
        bucket_pass<SampleKeys<THREADS>, THREADS, kSampleBuckets>(sample, smin, smax, shift, 0, r0, r1, sh);
        const uint32_t b0 = sh.result[0], b1 = sh.result[3];
        __syncthreads();
        // Ranks at the sample's ends open the range to the whole key space.
        p_lo = r0 == 0 ? 0u : smin + (b0 << shift);
        const uint64_t top = static_cast<uint64_t>(smin) + ((static_cast<uint64_t>(b1) + 1) << shift) - 1;
        p_hi = r1 == m - 1 ? 0xffffffffu : static_cast<uint32_t>(top < smax ? top : smax);
    }
    if (blockIdx.x == 0 && tid == 0) {
        header[0] = p_lo;
        header[1] = p_hi;
    }

    // Classify own scores; decided mask bytes are written now.
    uint32_t below = 0, nan = 0, cand = 0, cand_bits = 0, out = 0, cmin = 0xffffffffu, cmax = 0;
#pragma unroll
    for (int c = 0; c < kPartPerThread; ++c) {
        if (base + c >= n) continue;
        const uint32_t k = order_key(v[c]);
        if (v[c] != v[c]) {
            ++nan;
        } else if (k < p_lo) {
            ++below;
        } else if (k > p_hi) {
            out |= ((vw >> (8 * c)) & 0xffu ? 1u : 0u) << (8 * c);
        } else {
            ++cand;
            cand_bits |= 1u << c;
            cmin = min(cmin, k);
            cmax = max(cmax, k);
        }
    }
    if constexpr (VEC) {
        if (base < n) *reinterpret_cast<uint32_t*>(adm + base) = out;
    } else {
#pragma unroll
        for (int c = 0; c < kPartPerThread; ++c)
            if (base + c < n && !((cand_bits >> c) & 1u)) adm[base + c] = static_cast<uint8_t>((out >> (8 * c)) & 0xffu);
    }
    // Exclusive scan of the candidate counts over the workgroup; totals.
    const int lane = lane_id(), w = tid / kWave;
    uint32_t incl = cand;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t up = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += up;
    }
    uint32_t below_sum = below, nan_sum = nan;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        below_sum += __shfl_xor(below_sum, off, kWave);
        nan_sum += __shfl_xor(nan_sum, off, kWave);
        cmin = min(cmin, static_cast<uint32_t>(__shfl_xor(cmin, off, kWave)));
        cmax = max(cmax, static_cast<uint32_t>(__shfl_xor(cmax, off, kWave)));
    }
    if (lane == kWave - 1) sh.wave_tmp[0][w] = incl;
    if (lane == 0) {
        sh.wave_tmp[1][w] = below_sum;
        sh.wave_tmp[2][w] = nan_sum;
        sh.list[0][w] = cmin;
        sh.list[1][w] = cmax;
    }
    __syncthreads();
    uint32_t pos = incl - cand, total = 0, below_total = 0, nan_total = 0;
    cmin = 0xffffffffu;
    cmax = 0;
#pragma unroll
    for (int i = 0; i < THREADS / kWave; ++i) {
        if (i < w) pos += sh.wave_tmp[0][i];
        total += sh.wave_tmp[0][i];
        below_total += sh.wave_tmp[1][i];
        nan_total += sh.wave_tmp[2][i];
        cmin = min(cmin, sh.list[0][i]);
        cmax = max(cmax, sh.list[1][i]);
    }
    uint32_t* keys_out = cand_key + static_cast<int64_t>(blockIdx.x) * kCand;
    uint32_t* index_out = cand_index + static_cast<int64_t>(blockIdx.x) * kCand;
#pragma unroll
    for (int c = 0; c < kPartPerThread; ++c) {
        if ((cand_bits >> c) & 1u) {
            if (pos < kCand) {
                keys_out[pos] = order_key(v[c]);
                const uint32_t ok = ((vw >> (8 * c)) & 0xffu) ? 0x80000000u : 0u;
                index_out[pos] = static_cast<uint32_t>(tid * kPartPerThread + c) | ok;
            }
            ++pos;
        }
    }
    if (tid == 0) {
        uint32_t* rec = records + static_cast<int64_t>(blockIdx.x) * kRecordWords;
        rec[0] = below_total;
        rec[1] = total;
        rec[2] = nan_total;
        rec[3] = cmin;
        rec[4] = cmax;
    }
}

// Candidate keys gathered in LDS.
template <int THREADS>
struct LdsKeys {
    const uint32_t* key;
    uint32_t m;
    template <class F>
    __device__ void visit(F f) const {
        for (uint32_t i = threadIdx.x; i < m; i += THREADS) f(key[i]);
    }
    template <class F>
    __device__ void visit_all(F f) const {
        visit([&](uint32_t k) { f(k, true); });
    }
};

// SLOT: candidate slots per partition workgroup (its thread count), GMAX:
// the most workgroups this instance reads. Flat slot entry f = g * SLOT + e is
// loaded by thread f % kSelThreads (E = GMAX * SLOT / kSelThreads per thread).
template <int SLOT, int GMAX>
__global__ __launch_bounds__(kSelThreads) void quantile_finish_kernel(
    const float* __restrict__ s, const uint8_t* __restrict__ valid, uint8_t* __restrict__ adm,
    float* __restrict__ tau_out, int64_t n, int64_t k_lo, int64_t k_hi, float weight,
    const uint32_t* __restrict__ header, const uint32_t* __restrict__ records, const uint32_t* __restrict__ cand_key,
    const uint32_t* __restrict__ cand_index, int groups) {
    constexpr int THREADS = kSelThreads;
    constexpr int kScores = SLOT * kPartPerThread;  // scores per partition workgroup
    constexpr int E = GMAX * SLOT / THREADS;
    static_assert(E >= 1 && GMAX * SLOT % THREADS == 0 && GMAX <= kWave, "slot entry layout");
    __shared__ SelShared sh;
    __shared__ uint32_t keys[kFinishCand];
    const int tid = threadIdx.x;
    // One round trip: lane g of every wave loads record g (vector loads, all in
    // flight together), every thread loads its E slot entries (in bounds
    // whatever the counts), and the pivots. Totals, the candidates' key range
    // and each slot's offset among the gathered candidates come from the
    // records by wave reductions and a wave scan (no barrier).
    const int lane = lane_id();
    const int rg = lane < groups ? lane : groups - 1;
    const uint32_t* rec = records + rg * kRecordWords;
    uint32_t rec_below = rec[0], rec_cand = rec[1], rec_nan = rec[2], rec_min = rec[3], rec_max = rec[4];
    uint32_t key[E], index[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const int f = tid + k * THREADS;
        const int g = f / SLOT;
        const int gc = g < groups ? g : groups - 1;
        key[k] = cand_key[static_cast<int64_t>(gc) * SLOT + f % SLOT];
        index[k] = cand_index[static_cast<int64_t>(gc) * SLOT + f % SLOT];
    }
    if (lane >= groups) {
        rec_below = rec_cand = rec_nan = 0;
        rec_min = 0xffffffffu;
        rec_max = 0;
    }
    uint32_t below = rec_below, cand = rec_cand, bad = (rec_nan != 0 || rec_cand > SLOT) ? 1u : 0u;
    uint32_t kmin = rec_min, kmax = rec_max;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        below += __shfl_xor(below, off, kWave);
        cand += __shfl_xor(cand, off, kWave);
        bad |= __shfl_xor(bad, off, kWave);
        kmin = min(kmin, static_cast<uint32_t>(__shfl_xor(kmin, off, kWave)));
        kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(kmax, off, kWave)));
    }
    uint32_t prefix = rec_cand;  // inclusive scan of the slot counts over the lanes
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t up = __shfl_up(prefix, off, kWave);
        if (lane >= off) prefix += up;
    }
    prefix -= rec_cand;
    // A wave's 64 entries lie in one slot (SLOT % 64 == 0), so each slot's count
    // and offset are wave-uniform (scalar registers).
    static_assert(SLOT % kWave == 0, "one slot per wave and entry");
    uint32_t count[E], offset[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
        const int g = __builtin_amdgcn_readfirstlane((tid + k * THREADS) / SLOT);  // < GMAX; count 0 past `groups`
        count[k] = __builtin_amdgcn_readlane(rec_cand, g);
        offset[k] = __builtin_amdgcn_readlane(prefix, g);
    }
    const uint32_t p_lo = header[0], p_hi = header[1];
    const bool fast = bad == 0 && cand <= kFinishCand && static_cast<int64_t>(below) <= k_lo &&
                      k_hi < static_cast<int64_t>(below) + static_cast<int64_t>(cand);
    float tau = 0.0f;
    bool decided = false;
    if (fast) {
#pragma unroll
        for (int k = 0; k < E; ++k) {
            const uint32_t e = static_cast<uint32_t>((tid + k * THREADS) % SLOT);
            if (e < count[k]) keys[offset[k] + e] = key[k];
        }
        __syncthreads();
        LdsKeys<THREADS> lk{keys, cand};
        uint32_t key_lo, key_hi;
        select_two_ranks<LdsKeys<THREADS>, 10, THREADS>(lk, kmin, kmax, static_cast<uint32_t>(k_lo - below),
                                                        static_cast<uint32_t>(k_hi - below), sh, key_lo, key_hi);
        const float v_lo = key_to_float(key_lo);
        const float v_hi = key_to_float(key_hi);
        tau = weight < 0.5f ? __builtin_fmaf(weight, v_hi - v_lo, v_lo)
                            : __builtin_fmaf(weight - 1.0f, v_hi - v_lo, v_hi);
        // Every decided byte is right when tau lies in [p_lo, p_hi]; for tau = ±0
        // both zero keys must lie inside too (+0 > -0 is false for floats).
        const uint32_t tk = order_key(tau);
        decided = tau == tau && tk >= p_lo && tk <= p_hi;
        if (tau == 0.0f) decided = decided && order_key(-0.0f) >= p_lo && order_key(0.0f) <= p_hi;
        if (decided) {
            // Mask bytes of the candidates (every other byte was decided by the partition).
#pragma unroll
            for (int k = 0; k < E; ++k) {
                const int f = tid + k * THREADS;
                if (static_cast<uint32_t>(f % SLOT) < count[k]) {
                    const int64_t i = static_cast<int64_t>(f / SLOT) * kScores + (index[k] & 0x7fffffffu);
                    adm[i] = ((index[k] >> 31) && key_to_float(key[k]) > tau) ? 1 : 0;
                }
            }
        }
    }
    if (!decided) {
        // Exact select over all scores from memory, and the whole mask.
        MemoryKeys<THREADS> mk;
        mk.load(s, valid, n);
        uint32_t counted = 0, kmin = 0xffffffffu, kmax = 0;
        mk.visit([&](uint32_t k) {
            ++counted;
            kmin = min(kmin, k);
            kmax = max(kmax, k);
        });
        block_count_min_max<THREADS>(counted, kmin, kmax, sh);
        if (static_cast<int64_t>(counted) != n) {
            tau = __builtin_nanf("");
        } else {
            uint32_t key_lo, key_hi;
            select_two_ranks<MemoryKeys<THREADS>, 12, THREADS>(mk, kmin, kmax, static_cast<uint32_t>(k_lo),
                                                               static_cast<uint32_t>(k_hi), sh, key_lo, key_hi);
            const float v_lo = key_to_float(key_lo);
            const float v_hi = key_to_float(key_hi);
            tau = weight < 0.5f ? __builtin_fmaf(weight, v_hi - v_lo, v_lo)
                                : __builtin_fmaf(weight - 1.0f, v_hi - v_lo, v_hi);
        }
        mk.write_mask(adm, n, tau);
    }
    if (tid == 0) *tau_out = tau;
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
        const dim3 grid(grid_for(rows, kRowWaves * 4));
        auto launch16 = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, block, 0, stream, logits, b, targets, valid, o, rows, V, log_vocab,
                               static_cast<const float*>(nullptr), int64_t(1), static_cast<uint8_t*>(nullptr), 0.0f,
                               LayerBias<T>{}, int64_t(1));
        };
        if (vec && V == 256) {
            if (b) launch16(surprise_rows16_kernel<T, true, true, true>);
            else launch16(surprise_rows16_kernel<T, true, false, true>);
        } else if (vec) {
            if (b) launch16(surprise_rows16_kernel<T, true, true, false>);
            else launch16(surprise_rows16_kernel<T, true, false, false>);
        } else {
            if (b) launch16(surprise_rows16_kernel<T, false, true, false>);
            else launch16(surprise_rows16_kernel<T, false, false, false>);
        }
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

extern "C" int koemi_herm_surprise_shifted(const float* logits, const float* first, const float* bias,
                                           const int64_t* target_ids, const uint8_t* valid_mask, float* surprise,
                                           uint8_t* admission, float threshold, int64_t batch, int64_t length,
                                           int64_t vocab, float log_vocab, koemi_stream_t stream) {
    if (batch < 0 || length < 1 || vocab < 1) return fail(KOEMI_ERR_INVALID, "shifted surprise needs length, vocab >= 1");
    if (vocab != 256) return fail(KOEMI_ERR_UNSUPPORTED, "shifted surprise supports a content vocabulary of 256");
    if (batch == 0) return KOEMI_OK;
    if (!logits || !first || !target_ids || !valid_mask || !surprise)
        return fail(KOEMI_ERR_INVALID, "shifted surprise received a null pointer");
    if (reinterpret_cast<uintptr_t>(logits) % 16 != 0 || reinterpret_cast<uintptr_t>(first) % 16 != 0)
        return fail(KOEMI_ERR_INVALID, "shifted surprise needs 16-byte aligned logits");
    const int64_t rows = batch * length;
    const dim3 grid(grid_for(rows, kRowWaves * 4));
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(kWave * kRowWaves), 0, as_stream(stream), logits, bias, target_ids,
                           valid_mask, surprise, rows, vocab, log_vocab, first, length, admission, threshold,
                           LayerBias<float>{}, int64_t(1));
    };
    if (bias) launch(surprise_rows16_kernel<float, true, true, true, true>);
    else launch(surprise_rows16_kernel<float, true, false, true, true>);
    return check_launch("koemi_herm_surprise_shifted");
}

extern "C" int koemi_herm_surprise_layers(const float* logits, const float* const* biases,
                                          const int64_t* target_ids, const uint8_t* valid_mask, float* surprise,
                                          uint8_t* admission, float threshold, int layers, int64_t batch,
                                          int64_t vocab, float log_vocab, koemi_stream_t stream) {
    if (batch < 0 || layers < 1 || vocab < 1)
        return fail(KOEMI_ERR_INVALID, "layered surprise needs batch >= 0, layers and vocab >= 1");
    if (vocab != 256) return fail(KOEMI_ERR_UNSUPPORTED, "layered surprise supports a content vocabulary of 256");
    if (layers > kMaxLayers) return fail(KOEMI_ERR_UNSUPPORTED, "layered surprise takes at most %d layers", kMaxLayers);
    if (batch == 0) return KOEMI_OK;
    if (!logits || !biases || !target_ids || !valid_mask || !surprise)
        return fail(KOEMI_ERR_INVALID, "layered surprise received a null pointer");
    if (reinterpret_cast<uintptr_t>(logits) % 16 != 0)
        return fail(KOEMI_ERR_INVALID, "layered surprise needs 16-byte aligned logits");
    LayerBias<float> lb{};
    for (int l = 0; l < layers; ++l) {
        if (!biases[l]) return fail(KOEMI_ERR_INVALID, "layered surprise: bias %d is null", l);
        lb.p[l] = biases[l];
    }
    const int64_t rows = batch * layers;
    const dim3 grid(grid_for(rows, kRowWaves * 4));
    hipLaunchKernelGGL((surprise_rows16_kernel<float, true, true, true, true, true>), grid, dim3(kWave * kRowWaves), 0,
                       as_stream(stream), logits, nullptr, target_ids, valid_mask, surprise, rows, vocab, log_vocab,
                       logits, int64_t{1}, admission, threshold, lb, batch);
    return check_launch("koemi_herm_surprise_layers");
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

// Inputs handled by the two-kernel path (more use the single workgroup).
inline bool partitioned(int64_t count) {
    return count > kPartitionMin && count <= kPartMax;
}

namespace {

// The no-alloc entry point's workspace: one static device array per GPU, sized
// for the largest partitioned input (32 workgroup records and 2 x 32 x 1024
// candidate slots: 257 KiB). Inputs outside the partitioned range need no
// workspace, so every count fits.
constexpr size_t kQuantileScratchBytes = 256 + ((size_t(kPartMaxGroups) * kRecordWords * 4 + 255) & ~size_t(255)) +
                                         2 * ((size_t(kPartMaxGroups) * 1024 * 4 + 255) & ~size_t(255));
__device__ __align__(256) uint8_t scratch[kQuantileScratchBytes];

// Device address of `scratch` on each GPU, resolved once per device (with the
// device current) by the first no-alloc call there. In host code `scratch`
// names a host-side stand-in, never the device memory: only these addresses
// are passed to kernels.
constexpr int kMaxScratchDevices = 64;
std::once_flag g_scratch_once[kMaxScratchDevices];
void* g_scratch_ptr[kMaxScratchDevices];
hipError_t g_scratch_status[kMaxScratchDevices];

int scratch_for_current_device(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        return fail(KOEMI_ERR_LAUNCH, "quantile admission (no alloc): no current device");
    if (dev >= kMaxScratchDevices)
        return fail(KOEMI_ERR_UNSUPPORTED, "quantile admission (no alloc): device %d beyond the %d supported", dev,
                    kMaxScratchDevices);
    std::call_once(g_scratch_once[dev], [dev] {
        void* p = nullptr;
        g_scratch_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = p;
    });
    if (g_scratch_status[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr)
        return fail(KOEMI_ERR_LAUNCH, "quantile admission (no alloc): hipGetSymbolAddress failed on device %d (%s)", dev,
                    hipGetErrorString(g_scratch_status[dev]));
    *out = g_scratch_ptr[dev];
    return KOEMI_OK;
}

}  // namespace

extern "C" size_t koemi_admission_quantile_workspace_bytes(int64_t count) {
    if (!partitioned(count)) return 0;
    return part_workspace(count).total;
}

extern "C" int koemi_admission_quantile_noalloc(const float* surprise, const uint8_t* valid_mask,
                                                uint8_t* admission, float* threshold_out, int64_t count,
                                                float quantile, koemi_stream_t stream) {
    if (count < 1) return fail(KOEMI_ERR_INVALID, "quantile admission needs at least one score");
    if (count > 0xffffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "quantile admission supports at most 2^32-1 scores");
    const size_t need = partitioned(count) ? part_workspace(count).total : 0;
    if (need > kQuantileScratchBytes)
        return fail(KOEMI_ERR_UNSUPPORTED, "quantile admission (no alloc): %zu workspace bytes exceed the %zu-byte "
                    "static scratch", need, kQuantileScratchBytes);
    void* ws = nullptr;
    if (need) {
        const int st = scratch_for_current_device(&ws);
        if (st != KOEMI_OK) return st;
    }
    return koemi_admission_quantile(surprise, valid_mask, admission, threshold_out, count, quantile, ws,
                                    need ? kQuantileScratchBytes : 0, stream);
}

extern "C" int koemi_admission_quantile(const float* surprise, const uint8_t* valid_mask,
                                        uint8_t* admission, float* threshold_out, int64_t count,
                                        float quantile, void* workspace, size_t workspace_bytes,
                                        koemi_stream_t stream) {
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
    const bool vec = count % 4 == 0 && reinterpret_cast<uintptr_t>(surprise) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(valid_mask) % 4 == 0 && reinterpret_cast<uintptr_t>(admission) % 4 == 0;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(1), dim3(kSelThreads), 0, s, surprise, valid_mask, admission, threshold_out,
                           count, k_lo, k_hi, weight);
    };
    if (count <= kPartitionMin) {
        if (vec) launch(quantile_admission_kernel<RegisterKeys<8, true>>);
        else launch(quantile_admission_kernel<RegisterKeys<8, false>>);
        return check_launch("koemi_admission_quantile");
    }
    if (!partitioned(count)) {
        launch(quantile_admission_kernel<MemoryKeys<kSelThreads>>);
        return check_launch("koemi_admission_quantile");
    }
    const PartWorkspace pw = part_workspace(count);
    if (!workspace || workspace_bytes < pw.total)
        return fail(KOEMI_ERR_INVALID, "quantile admission workspace too small: need %zu bytes", pw.total);
    const int groups = pw.groups;
    char* ws = static_cast<char*>(workspace);
    uint32_t* header = reinterpret_cast<uint32_t*>(ws + pw.header_off);
    uint32_t* records = reinterpret_cast<uint32_t*>(ws + pw.record_off);
    uint32_t* cand_key = reinterpret_cast<uint32_t*>(ws + pw.key_off);
    uint32_t* cand_index = reinterpret_cast<uint32_t*>(ws + pw.index_off);
    auto run = [&](auto threads_tag) -> int {
        constexpr int T = decltype(threads_tag)::value;
        auto partition = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(groups)), dim3(T), 0, s, surprise, valid_mask,
                               admission, count, k_lo, k_hi, header, records, cand_key, cand_index);
        };
        if (vec) partition(quantile_partition_kernel<T, true>);
        else partition(quantile_partition_kernel<T, false>);
        const int st = check_launch("koemi_admission_quantile(partition)");
        if (st != KOEMI_OK) return st;
        auto finish = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(1), dim3(kSelThreads), 0, s, surprise, valid_mask, admission,
                               threshold_out, count, k_lo, k_hi, weight, header, records, cand_key, cand_index, groups);
        };
        if (groups <= 8) finish(quantile_finish_kernel<T, 8>);
        else if (groups <= 16) finish(quantile_finish_kernel<T, 16>);
        else finish(quantile_finish_kernel<T, kPartMaxGroups>);
        return KOEMI_OK;
    };
    const int st = pw.threads == 256 ? run(std::integral_constant<int, 256>{})
                                     : run(std::integral_constant<int, 1024>{});
    if (st != KOEMI_OK) return st;
    return check_launch("koemi_admission_quantile");
}
