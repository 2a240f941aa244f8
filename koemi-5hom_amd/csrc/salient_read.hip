// Salient-memory read for gfx950.
//
// Reference: model/memory.py:405-429 (LocalKeyValueMemory.read_salient_window),
// called at network.py:350-358 with the window's working states as queries:
//
//   keys   = [carried_keys ; keys]                 [B, S + L, D]
//   score  = keys . query / sqrt(D)                [B, L, S + L]
//   slot s is eligible for query t when s < S and carried_valid[s], or
//   s = S + j with admission[j] and j < t (strictly earlier window positions);
//   weight = softmax over the eligible slots (all zero when none is), and
//   out    = weight . [carried_values ; values]    [B, L, D]
//
// Up to kFusedMaxSlots slots (S + L) two kernels on fp32 MFMA
// (v_mfma_f32_32x32x2f32), every operand converted to fp32:
//   scores: one workgroup per (32 slots, 32 queries, batch, half of the
//     width); its four waves split that half further, stage 32 x 64 slices of
//     queries and keys in LDS (rows padded to 66 floats: conflict-free operand
//     reads) and sum their partial 32 x 32 products through LDS. Slot tiles that
//     causality hides from every query of the tile are skipped.
//   read: one workgroup per (128 output columns, 32 queries, batch). Each
//     wave owns 8 query rows: it adds the two width halves of their scores,
//     masks them (eligibility from the valid and admission bytes and the
//     positions), takes the row maxima on the way and leaves exp(score - max)
//     in LDS with the row sums. Then each wave multiplies the 32 x K block of
//     exponentials with a 32-column slice of the values, read straight from
//     memory two 16-step windows ahead of use (each MFMA's value operand is two
//     128-byte row segments), and divides by the row sums on the way out
//     (all-zero rows when nothing is eligible).
// Longer slot axes use rocBLAS for the two products (fp32 accumulation; the
// carried and window parts of the key axis as separate strided-batched calls
// on the caller's tensors) around a masked-softmax kernel. rocBLAS is
// column-major: a row-major [rows, cols] matrix is its [cols, rows]
// column-major view, so score^T = K'^T Q' and out' = V' P'.
#include "common.hpp"

#include <rocblas/rocblas.h>

#include <cmath>
#include <mutex>

namespace koemi {

// The rocBLAS handle of a device (blas.hip); callers hold g_blas_mutex.
rocblas_handle blas_handle(int device);
extern std::mutex g_blas_mutex;

namespace {

constexpr int kSoftmaxWaves = 4;
constexpr int64_t kFusedMaxSlots = 1024;  // the read kernel keeps 32 rows of exponentials in LDS (32 x 1026 floats)
constexpr int kSplitD = 2;                // width halves of the scores kernel
constexpr int kPitch = 66;                // LDS row pitch (floats) of the scores kernel's operands

typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
__device__ __forceinline__ float load_f32(const T* p) {
    return to_f32(*p);
}

// Four consecutive elements as fp32 (16-byte loads for fp32, 8-byte otherwise;
// the caller guarantees the alignment: width % 4 == 0 and aligned rows).
template <typename T>
__device__ __forceinline__ float4 load4_f32(const T* p) {
    if constexpr (sizeof(T) == 4) {
        return *reinterpret_cast<const float4*>(p);
    } else {
        union {
            uint2 raw;
            T h[4];
        } u;
        u.raw = *reinterpret_cast<const uint2*>(p);
        return make_float4(to_f32(u.h[0]), to_f32(u.h[1]), to_f32(u.h[2]), to_f32(u.h[3]));
    }
}

// Scores of slots [s0, s0 + 32) for queries [q0, q0 + 32) of batch b over the
// width half h: scores[h][b][t][s] = (sum over the half of key_s . query_t) / sqrt(D).
// VEC: width % 4 == 0 (four-element loads).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void salient_scores_kernel(
    const T* __restrict__ ck, const T* __restrict__ k, const T* __restrict__ q, float* __restrict__ scores,
    int64_t B, int64_t S, int64_t L, int64_t D, float inv_sqrt_d) {
    __shared__ float stage[4][2][32 * kPitch];  // per wave: queries, keys (67.6 KiB: two workgroups per CU)
    const int64_t K = S + L;
    const int64_t s0 = static_cast<int64_t>(blockIdx.x) * 32, q0 = static_cast<int64_t>(blockIdx.y) * 32;
    const int64_t b = blockIdx.z / kSplitD;
    const int half = static_cast<int>(blockIdx.z % kSplitD);
    // Window slot j is seen by queries t > j only: skip tiles no query here sees.
    const int64_t t_max = min(q0 + 31, L - 1);
    if (s0 >= S && s0 - S >= t_max) return;
    const int lane = lane_id(), wave = threadIdx.x / kWave;
    // Halves start at multiples of 4, so with width % 4 == 0 every four-element
    // group lies inside one half and one row.
    const int64_t d_half = ((D + kSplitD - 1) / kSplitD + 3) & ~int64_t(3);
    const int64_t d_lo = min(D, half * d_half), d_hi = min(D, d_lo + d_half);
    const int64_t nchunks = (d_hi - d_lo + 63) / 64;
    // Lane l stages rows l / 16 + 4 i (i < 8), columns 4 (l % 16) .. +3 of a chunk.
    const T* qrow[8];
    const T* krow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = lane / 16 + 4 * i;
        const int64_t t = min(q0 + r, L - 1), sl = min(s0 + r, K - 1);
        qrow[i] = q + (b * L + t) * D;
        krow[i] = sl < S ? ck + (b * S + sl) * D : k + (b * L + (sl - S)) * D;
    }
    const int col = (lane % 16) * 4;
    float4 qv[8], kv[8];
    auto load_chunk = [&](int64_t c) {
        const int64_t d = d_lo + c * 64 + col;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (VEC) {
                const bool in = d < d_hi;
                const int64_t dc = in ? d : d_lo;  // d_lo and d_hi are multiples of 4 here
                qv[i] = load4_f32(qrow[i] + dc);
                kv[i] = load4_f32(krow[i] + dc);
                if (!in) qv[i] = kv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            } else {
                float a[4], e[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    const bool in = d + x < d_hi;
                    const int64_t dc = in ? d + x : d_lo;
                    a[x] = in ? load_f32(qrow[i] + dc) : 0.0f;
                    e[x] = in ? load_f32(krow[i] + dc) : 0.0f;
                }
                qv[i] = make_float4(a[0], a[1], a[2], a[3]);
                kv[i] = make_float4(e[0], e[1], e[2], e[3]);
            }
        }
    };
    auto store_chunk = [&]() {
        float* qs = stage[wave][0];
        float* ks = stage[wave][1];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = lane / 16 + 4 * i;
            // rows are 264 bytes apart: 8-byte aligned pairs
            *reinterpret_cast<float2*>(qs + r * kPitch + col) = make_float2(qv[i].x, qv[i].y);
            *reinterpret_cast<float2*>(qs + r * kPitch + col + 2) = make_float2(qv[i].z, qv[i].w);
            *reinterpret_cast<float2*>(ks + r * kPitch + col) = make_float2(kv[i].x, kv[i].y);
            *reinterpret_cast<float2*>(ks + r * kPitch + col + 2) = make_float2(kv[i].z, kv[i].w);
        }
    };
    // Two accumulators (even and odd K steps) keep two MFMA chains in flight.
    f32x16 acc0, acc1;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.0f;
    // Wave w takes chunks w, w + 4, ...; the next chunk's loads are in flight
    // (in registers) while the current one is multiplied from LDS. A wave's LDS
    // operations complete in order, so the next chunk's stores wait for this
    // chunk's operand reads.
    int64_t c = wave;
    if (c < nchunks) load_chunk(c);
    for (; c < nchunks; c += 4) {
        store_chunk();
        if (c + 4 < nchunks) load_chunk(c + 4);
        const float* qs = stage[wave][0];
        const float* ks = stage[wave][1];
        // Lane l: row l % 32 of each operand, K index 2 kk + l / 32; sixteen
        // operand pairs are read before their MFMAs (one LDS latency each).
#pragma unroll
        for (int kb = 0; kb < 32; kb += 16) {
            float a[16], e[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int idx = (lane % 32) * kPitch + 2 * (kb + i) + lane / 32;
                a[i] = qs[idx];
                e[i] = ks[idx];
            }
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], e[i], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i + 1], e[i + 1], acc1, 0, 0, 0);
            }
        }
    }
    f32x16 acc = acc0 + acc1;
    // Sum the four waves' partial tiles: element v of lane l is query
    // 8 (v / 4) + 4 (l / 32) + v % 4, slot l % 32.
    __syncthreads();
    float* red = &stage[0][0][0];  // 4 x 16 x 64 floats
#pragma unroll
    for (int v = 0; v < 16; ++v) red[(wave * 16 + v) * kWave + lane] = acc[v];
    __syncthreads();
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
        const int v = wave * 4 + vv;
        const float sum = red[(0 * 16 + v) * kWave + lane] + red[(1 * 16 + v) * kWave + lane] +
                          red[(2 * 16 + v) * kWave + lane] + red[(3 * 16 + v) * kWave + lane];
        const int64_t t = q0 + 8 * (v / 4) + 4 * (lane / 32) + v % 4;
        const int64_t sl = s0 + lane % 32;
        if (t < L && sl < K) scores[((half * B + b) * L + t) * K + sl] = sum * inv_sqrt_d;
    }
}

// out[b][t][d] for queries [q0, q0 + 32) and columns [d0, d0 + 128).
template <typename T>
__global__ __launch_bounds__(256) void salient_read_kernel(
    const float* __restrict__ scores, const uint8_t* __restrict__ carried_valid, const uint8_t* __restrict__ admission,
    const T* __restrict__ cv, const T* __restrict__ v, T* __restrict__ out, int64_t B, int64_t S, int64_t L,
    int64_t D, int pitch) {
    extern __shared__ float p_sh[];  // 32 x pitch exponentials, then the 32 rows' sums
    float* row_sum = p_sh + 32 * pitch;
    // Slot and row indices fit 32 bits (S + L <= kFusedMaxSlots); memory offsets are 64-bit.
    const int K = static_cast<int>(S + L), Si = static_cast<int>(S), Li = static_cast<int>(L);
    const int64_t d0 = static_cast<int64_t>(blockIdx.x) * 128;
    const int q0 = static_cast<int>(blockIdx.y) * 32;
    const int64_t b = blockIdx.z;
    const int lane = lane_id(), wave = static_cast<int>(threadIdx.x) / kWave;

    // Wave w computes columns dw .. dw + 31 of out = E (32 x K) . V (K x 32) in
    // steps of two slots, windows of 16 steps; the value rows of its first two
    // windows are requested before the softmax, and every later window two
    // windows ahead of its use.
    const int64_t dw = d0 + wave * 32;
    const int64_t dcol = min(dw + lane % 32, D - 1);
    const T* cv_b = cv + b * S * D + dcol;  // + slot * D (carried slots)
    const T* v_b = v + b * L * D + dcol;    // + (slot - S) * D (window slots)
    const int windows = ((K + 1) / 2 + 15) / 16;
    auto vwindow = [&](float(&dst)[16], int w) {
        if (w >= windows) return;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int sl = min(32 * w + 2 * i + lane / 32, K - 1);  // clamped rows carry zero weight
            dst[i] = load_f32(sl < Si ? cv_b + static_cast<int64_t>(sl) * D : v_b + static_cast<int64_t>(sl - Si) * D);
        }
    };
    float va[16], vb[16], vc[16];
    vwindow(va, 0);
    vwindow(vb, 1);

    // Wave w owns query rows r0 .. r0 + 7 (r0 = 8 w) of the tile: it adds the
    // two width halves of their scores, keeps the eligible ones (-inf
    // elsewhere) in LDS and takes their maxima on the way, 2 x 64 slots per
    // round trip. Slot sl is eligible for query t < L when its valid or
    // admission byte is set and sl < S + t.
    const int r0 = wave * 8;
    const float* half0 = scores + b * L * K;
    const float* half1 = half0 + B * L * K;
    int lim[8], row_off[8];
    float m[8];
    bool any[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const int t = q0 + r0 + r;
        lim[r] = t < Li ? Si + t : 0;
        row_off[r] = min(t, Li - 1) * K;
        m[r] = -INFINITY;
        any[r] = false;
    }
    for (int c = 0; c < K; c += 128) {
        float x0[2][8], x1[2][8];
        bool f[2];
        int col[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            col[j] = c + 64 * j + lane;
            const int sl = min(col[j], K - 1);
            f[j] = (sl < Si ? carried_valid[b * S + sl] : admission[b * L + (sl - Si)]) != 0;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                x0[j][r] = half0[row_off[r] + sl];
                x1[j][r] = half1[row_off[r] + sl];
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (col[j] >= K) continue;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const bool ok = f[j] && col[j] < lim[r];
                const float x = x0[j][r] + x1[j][r];
                p_sh[(r0 + r) * pitch + col[j]] = ok ? x : -INFINITY;
                if (ok) {
                    any[r] = true;
                    m[r] = fmaxf(m[r], x);
                }
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < 8; ++r) m[r] = fmaxf(m[r], __shfl_xor(m[r], off, kWave));
    // Exponentials in place (zero past K up to the pitch, and in rows with no
    // eligible slot); the row sums divide the products at the end. Each lane
    // reads back only the cells it wrote.
    float sum[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        any[r] = __any(any[r]);
        if (!any[r]) m[r] = 0.0f;
        sum[r] = 0.0f;
    }
    for (int sl = lane; sl < pitch; sl += kWave) {
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            float* cell = p_sh + (r0 + r) * pitch + sl;
            const float e = sl < K ? expf(*cell - m[r]) : 0.0f;  // exp(-inf) = 0 for ineligible slots
            *cell = e;
            sum[r] += e;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
#pragma unroll
        for (int r = 0; r < 8; ++r) sum[r] += __shfl_xor(sum[r], off, kWave);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 8; ++r) row_sum[r0 + r] = sum[r];
    }
    __syncthreads();

    // E . V: the exponentials of 16 steps are read before their MFMAs; two
    // accumulators; the steps run to whole windows over the zero exponentials
    // that pad each row.
    f32x16 acc0, acc1;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.0f;
    const float* erow = p_sh + (lane % 32) * pitch + lane / 32;
    auto multiply = [&](const float(&vw)[16], int w) {
        float ew[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) ew[i] = erow[32 * w + 2 * i];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(ew[i], vw[i], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(ew[i + 1], vw[i + 1], acc1, 0, 0, 0);
        }
    };
    for (int w = 0; w < windows; w += 3) {
        vwindow(vc, w + 2);
        multiply(va, w);
        if (w + 1 >= windows) break;
        vwindow(va, w + 3);
        multiply(vb, w + 1);
        if (w + 2 >= windows) break;
        vwindow(vb, w + 4);
        multiply(vc, w + 2);
    }
    const f32x16 acc = acc0 + acc1;
    // Element i of lane l: query 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32;
    // a row whose exponentials sum to zero reads zeros.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = 8 * (i / 4) + 4 * (lane / 32) + i % 4;
        const int t = q0 + r;
        const int64_t d = dw + lane % 32;
        const float total = row_sum[r];
        const float o = total == 0.0f ? 0.0f : acc[i] / total;  // a NaN sum stays NaN
        if (t < Li && d < D) out[(b * L + t) * D + d] = from_f32<T>(o);
    }
}

// Row pitch (floats) of the read kernel's LDS weights: K rounded up to a
// multiple of 32 (the MFMA loop runs 16 two-slot steps at a time over the zero
// padding), plus 2 so that pitch / 2 is odd and the 32 rows of a column fall in
// distinct banks (the odd column of each pair in the other half of the banks).
inline int read_pitch(int64_t K) { return static_cast<int>((K + 31) / 32 * 32 + 2); }

template <typename T>
__global__ __launch_bounds__(kWave * kSoftmaxWaves) void masked_softmax_kernel(
    const float* __restrict__ score, const uint8_t* __restrict__ carried_valid, const uint8_t* __restrict__ admission,
    T* __restrict__ weight, int64_t B, int64_t S, int64_t L) {
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kSoftmaxWaves + threadIdx.x / kWave;  // b * L + t
    if (row >= B * L) return;
    const int64_t b = row / L, t = row % L;
    const int64_t K = S + L;
    const float* x = score + row * K;
    T* w = weight + row * K;
    auto eligible = [&](int64_t s) -> bool {
        if (s < S) return carried_valid[b * S + s] != 0;
        const int64_t j = s - S;
        return j < t && admission[b * L + j] != 0;
    };
    float m = -INFINITY;
    bool any = false;
    for (int64_t s = lane; s < K; s += kWave) {
        if (eligible(s)) {
            any = true;
            m = fmaxf(m, x[s]);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    any = __any(any);
    if (!any) {  // no eligible slot: the reference's torch.where gives zero weights
        for (int64_t s = lane; s < K; s += kWave) w[s] = from_f32<T>(0.0f);
        return;
    }
    float sum = 0.0f;
    for (int64_t s = lane; s < K; s += kWave)
        if (eligible(s)) sum += expf(x[s] - m);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
    const float inv = 1.0f / sum;
    for (int64_t s = lane; s < K; s += kWave) w[s] = from_f32<T>(eligible(s) ? expf(x[s] - m) * inv : 0.0f);
}

template <typename T>
__global__ void fp32_to_dtype_kernel(const float* __restrict__ src, T* __restrict__ dst, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = from_f32<T>(src[i]);
}

rocblas_datatype blas_type(int dtype) {
    switch (dtype) {
        case KOEMI_F16: return rocblas_datatype_f16_r;
        case KOEMI_BF16: return rocblas_datatype_bf16_r;
        default: return rocblas_datatype_f32_r;
    }
}

struct ReadWorkspace {
    size_t score_off, weight_off, out_off, total;
};
ReadWorkspace read_workspace(int64_t B, int64_t S, int64_t L, int64_t D, int dtype) {
    auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
    const size_t rows = static_cast<size_t>(B) * static_cast<size_t>(L);
    const size_t scores = rows * static_cast<size_t>(S + L);
    ReadWorkspace w;
    w.score_off = 0;
    if (S + L <= kFusedMaxSlots) {  // fused kernels: the two width halves of the scores
        w.weight_off = w.out_off = w.total = align(kSplitD * scores * sizeof(float));
    } else if (dtype == KOEMI_F32) {
        // The weights overwrite the scores (a lane reads each element before
        // writing it) and the second product writes the output directly.
        w.weight_off = w.score_off;
        w.out_off = w.total = align(scores * sizeof(float));
    } else {
        // Weights in the input dtype; the fp32 output is converted at the end.
        w.weight_off = align(scores * sizeof(float));
        w.out_off = w.weight_off + align(scores * 2);
        w.total = w.out_off + align(rows * static_cast<size_t>(D) * sizeof(float));
    }
    return w;
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" size_t koemi_salient_read_workspace_bytes(int64_t batch, int64_t carried, int64_t length, int64_t width,
                                                     int dtype) {
    if (batch < 0 || carried < 0 || length < 0 || width < 1) return 0;
    return read_workspace(batch, carried, length, width, dtype).total;
}

extern "C" int koemi_salient_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                                  const void* keys, const void* values, const uint8_t* admission, const void* queries,
                                  void* out, int64_t batch, int64_t carried, int64_t length, int64_t width, int dtype,
                                  void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || carried < 0 || length < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "salient read needs non-negative batch, carried and length and positive width");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "salient read does not support dtype %s", dtype_name(dtype));
    if (batch == 0 || length == 0) return KOEMI_OK;
    const int64_t K = carried + length;
    const int64_t limit = 0x7fffffffLL;
    if (K > limit || width > limit || length * K > limit || length * width > limit || K * width > limit ||
        batch * length > limit)
        return fail(KOEMI_ERR_UNSUPPORTED, "salient read sizes exceed 32-bit GEMM strides");
    if (!keys || !values || !admission || !queries || !out ||
        (carried > 0 && (!carried_keys || !carried_values || !carried_valid)))
        return fail(KOEMI_ERR_INVALID, "salient read received a null pointer");
    const ReadWorkspace ws = read_workspace(batch, carried, length, width, dtype);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "salient read workspace too small: need %zu bytes", ws.total);
    char* base = static_cast<char*>(workspace);
    float* score = reinterpret_cast<float*>(base + ws.score_off);
    void* weight = base + ws.weight_off;
    const hipStream_t s = as_stream(stream);

    if (K <= kFusedMaxSlots) {
        if (batch > 65535 / kSplitD || (length + 31) / 32 > 65535 || (width + 127) / 128 > 0x7fffffffLL)
            return fail(KOEMI_ERR_UNSUPPORTED, "salient read grid too large");
        const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
        const dim3 g1(static_cast<unsigned>((K + 31) / 32), static_cast<unsigned>((length + 31) / 32),
                      static_cast<unsigned>(batch * kSplitD));
        const dim3 g2(static_cast<unsigned>((width + 127) / 128), static_cast<unsigned>((length + 31) / 32),
                      static_cast<unsigned>(batch));
        const int pitch = read_pitch(K);
        const size_t lds = static_cast<size_t>(32) * (pitch + 1) * sizeof(float);
        const size_t esize = dtype == KOEMI_F32 ? 4 : 2;
        const bool vec = width % 4 == 0 && reinterpret_cast<uintptr_t>(queries) % (4 * esize) == 0 &&
                         reinterpret_cast<uintptr_t>(keys) % (4 * esize) == 0 &&
                         (carried == 0 || reinterpret_cast<uintptr_t>(carried_keys) % (4 * esize) == 0);
        auto run = [&](auto tag) {
            using T = decltype(tag);
            auto scores_kernel = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, g1, dim3(256), 0, s, static_cast<const T*>(carried_keys),
                                   static_cast<const T*>(keys), static_cast<const T*>(queries), score, batch, carried,
                                   length, width, inv_sqrt_d);
            };
            if (vec) scores_kernel(salient_scores_kernel<T, true>);
            else scores_kernel(salient_scores_kernel<T, false>);
            hipLaunchKernelGGL(salient_read_kernel<T>, g2, dim3(256), lds, s, score, carried_valid, admission,
                               static_cast<const T*>(carried_values), static_cast<const T*>(values),
                               static_cast<T*>(out), batch, carried, length, width, pitch);
        };
        if (dtype == KOEMI_F32) run(float{});
        else if (dtype == KOEMI_F16) run(f16{});
        else run(bf16{});
        return check_launch("koemi_salient_read");
    }

    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(KOEMI_ERR_LAUNCH, "salient read: no device");
    std::lock_guard<std::mutex> lock(g_blas_mutex);
    rocblas_handle h = blas_handle(dev);
    if (!h) return fail(KOEMI_ERR_LAUNCH, "salient read: no rocBLAS handle");
    if (rocblas_set_stream(h, s) != rocblas_status_success ||
        rocblas_set_pointer_mode(h, rocblas_pointer_mode_host) != rocblas_status_success)
        return fail(KOEMI_ERR_LAUNCH, "salient read: rocblas stream setup failed");
    const rocblas_datatype in_t = blas_type(dtype);
    const rocblas_int n = static_cast<rocblas_int>(length), d = static_cast<rocblas_int>(width);
    const rocblas_int kk = static_cast<rocblas_int>(K), S = static_cast<rocblas_int>(carried);
    const rocblas_int nb = static_cast<rocblas_int>(batch);
    const float scale = 1.0f / std::sqrt(static_cast<float>(width)), one = 1.0f, zero = 0.0f;
    const size_t esize = dtype == KOEMI_F32 ? 4 : 2;
    auto check = [](rocblas_status st, const char* what) {
        return st == rocblas_status_success ? KOEMI_OK : fail(KOEMI_ERR_LAUNCH, "salient read: %s failed (%s)", what,
                                                              rocblas_status_to_string(st));
    };

    // score^T[b] (K x L, ld K) = keys'^T (K x D) . queries' (D x L), scaled by 1/sqrt(D).
    int st = KOEMI_OK;
    if (carried > 0) {
        st = check(rocblas_gemm_strided_batched_ex(h, rocblas_operation_transpose, rocblas_operation_none, S, n, d,
                                                   &scale, carried_keys, in_t, d, static_cast<rocblas_stride>(S) * d,
                                                   queries, in_t, d, static_cast<rocblas_stride>(n) * d, &zero, score,
                                                   rocblas_datatype_f32_r, kk, static_cast<rocblas_stride>(n) * kk,
                                                   score, rocblas_datatype_f32_r, kk,
                                                   static_cast<rocblas_stride>(n) * kk, nb, rocblas_datatype_f32_r,
                                                   rocblas_gemm_algo_standard, 0, 0),
                   "carried scores");
        if (st != KOEMI_OK) return st;
    }
    st = check(rocblas_gemm_strided_batched_ex(h, rocblas_operation_transpose, rocblas_operation_none, n, n, d, &scale,
                                               keys, in_t, d, static_cast<rocblas_stride>(n) * d, queries, in_t, d,
                                               static_cast<rocblas_stride>(n) * d, &zero, score + carried,
                                               rocblas_datatype_f32_r, kk, static_cast<rocblas_stride>(n) * kk,
                                               score + carried, rocblas_datatype_f32_r, kk,
                                               static_cast<rocblas_stride>(n) * kk, nb, rocblas_datatype_f32_r,
                                               rocblas_gemm_algo_standard, 0, 0),
               "window scores");
    if (st != KOEMI_OK) return st;

    // Masked softmax over each query row; the weights go out in the input dtype.
    const int64_t rows = batch * length;
    const dim3 grid(static_cast<unsigned>((rows + kSoftmaxWaves - 1) / kSoftmaxWaves)), block(kWave * kSoftmaxWaves);
    switch (dtype) {
        case KOEMI_F32:
            hipLaunchKernelGGL(masked_softmax_kernel<float>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<float*>(weight), batch, carried, length);
            break;
        case KOEMI_F16:
            hipLaunchKernelGGL(masked_softmax_kernel<f16>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<f16*>(weight), batch, carried, length);
            break;
        default:
            hipLaunchKernelGGL(masked_softmax_kernel<bf16>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<bf16*>(weight), batch, carried, length);
    }
    st = check_launch("koemi_salient_read(softmax)");
    if (st != KOEMI_OK) return st;

    // out'[b] (D x L) = values' (D x K) . weight' (K x L): carried part, then the
    // window part accumulated on top (fp32 output; half dtypes are converted).
    float* acc = dtype == KOEMI_F32 ? static_cast<float*>(out) : reinterpret_cast<float*>(base + ws.out_off);
    const char* wbytes = static_cast<const char*>(weight);
    if (carried > 0) {
        st = check(rocblas_gemm_strided_batched_ex(h, rocblas_operation_none, rocblas_operation_none, d, n, S, &one,
                                                   carried_values, in_t, d, static_cast<rocblas_stride>(S) * d, wbytes,
                                                   in_t, kk, static_cast<rocblas_stride>(n) * kk, &zero, acc,
                                                   rocblas_datatype_f32_r, d, static_cast<rocblas_stride>(n) * d, acc,
                                                   rocblas_datatype_f32_r, d, static_cast<rocblas_stride>(n) * d, nb,
                                                   rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
                   "carried read");
        if (st != KOEMI_OK) return st;
    }
    st = check(rocblas_gemm_strided_batched_ex(h, rocblas_operation_none, rocblas_operation_none, d, n, n, &one,
                                               values, in_t, d, static_cast<rocblas_stride>(n) * d,
                                               wbytes + static_cast<size_t>(carried) * esize, in_t, kk,
                                               static_cast<rocblas_stride>(n) * kk, carried > 0 ? &one : &zero, acc,
                                               rocblas_datatype_f32_r, d, static_cast<rocblas_stride>(n) * d, acc,
                                               rocblas_datatype_f32_r, d, static_cast<rocblas_stride>(n) * d, nb,
                                               rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
               "window read");
    if (st != KOEMI_OK) return st;
    if (dtype != KOEMI_F32) {
        const int64_t total = rows * width;
        const dim3 g(static_cast<unsigned>((total + 255) / 256));
        if (dtype == KOEMI_F16)
            hipLaunchKernelGGL(fp32_to_dtype_kernel<f16>, g, dim3(256), 0, s, acc, static_cast<f16*>(out), total);
        else
            hipLaunchKernelGGL(fp32_to_dtype_kernel<bf16>, g, dim3(256), 0, s, acc, static_cast<bf16*>(out), total);
        return check_launch("koemi_salient_read(convert)");
    }
    return KOEMI_OK;
}
