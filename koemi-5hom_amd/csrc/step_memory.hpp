// The one-position (decode step) associative memory update shared by the
// associative memory's own launch and the decode step's combined memory
// launch.
#pragma once

#include "common.hpp"

namespace koemi {
namespace step {

constexpr float kMinDecay = 0.000244140625f;        // 2^-12
constexpr float kDecaySpan = 1.0f - 0.00048828125f;  // (1 - 2^-12) - 2^-12
constexpr float kReadEpsilon = 0.00390625f;          // 2^-8
constexpr float kMaxRefineDecay = 1.0f - 0.0000152587890625f;  // 1 - 2^-16 (memory.py:79)

// The refine memory's write terms (memory.py:257-268) of a position whose
// fast terms are (decay, weight before the surprise factor): decay' =
// min(1 - (1 - decay) rate, 1 - 2^-16), weight' = weight clamp(surprise, 0, 1)
// clamp(novelty, 0, 1); the value is clamp(value - fast read, -2, 2).
__device__ __forceinline__ float refine_decay(float decay, float rate) {
    return fminf(1.0f - (1.0f - decay) * rate, kMaxRefineDecay);
}
__device__ __forceinline__ float refine_value(float value, float fast) {
    return fminf(fmaxf(value - fast, -2.0f), 2.0f);
}

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// The associative memory of a one-position window (a decode step): the read
// from the carried state, then basis' = decay basis + weight value
// features^T and normalizer' likewise (memory.py:91-95, 279-288). Batch row
// b, columns [256 col_block, + 256), one thread per column (256 threads); the
// row's feature softmaxes and gates in LDS. With `novelty` (non-null: the
// refine memory of the herm ablation) the write terms are the refine terms
// (refine_decay, the weight times clamp(novelty), refine_value against the
// position's fast read `fast` [batch, D]).
template <int MAXM, typename PT>
__device__ __forceinline__ void assoc_step_body(
    const PT* __restrict__ proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
    int64_t decay_off, int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ out,
    float* __restrict__ next_basis, float* __restrict__ next_normalizer, int64_t D, int M, int64_t b,
    int col_block, const float* __restrict__ novelty = nullptr, float refine_rate = 0.0f,
    const float* __restrict__ fast = nullptr) {
    __shared__ float f_sh[MAXM], q_sh[MAXM], gate[3];  // decay, weight, normalizer . query features
    const int tid = threadIdx.x;
    const PT* row = proj + b * stride;
    if (tid < kWave) {
        // lanes 0..31: the key's feature softmax, lanes 32..63: the query's
        // (one feature per lane; max and sum by shuffles within each half)
        const int lane = tid, m = lane & 31;
        const bool query = lane >= 32, in = m < M;
        const float z = in ? to_f32(row[(query ? fq_off : fk_off) + min(m, M - 1)]) : -INFINITY;
        float mx = z;
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
        const float e = in ? expf(z - mx) : 0.0f;
        float sum = e;
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
        const float f = e / sum;
        if (m < MAXM) (query ? q_sh : f_sh)[m] = f;  // zero past M
        // normalizer . query features over the query half
        float nq = (query && in) ? normalizer[b * M + m] * f : 0.0f;
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) nq += __shfl_xor(nq, off, kWave);
        if (lane == 32) gate[2] = nq;
        if (lane == 0) {
            const bool ok = valid[b] != 0;
            const float sv = fminf(fmaxf(surprise[b], 0.0f), 1.0f);
            const float decay = kMinDecay + kDecaySpan * sigmoid_f(to_f32(row[decay_off]));
            const float wr = sigmoid_f(to_f32(row[write_off]));
            if (novelty != nullptr) {
                gate[0] = ok ? refine_decay(decay, refine_rate) : 1.0f;
                gate[1] = ok ? wr * sv * fminf(fmaxf(novelty[b], 0.0f), 1.0f) : 0.0f;
            } else {
                gate[0] = ok ? decay : 1.0f;
                gate[1] = ok ? wr * (0.25f + 0.75f * sv) : 0.0f;
            }
        }
    }
    __syncthreads();
    const float decay = gate[0], w = gate[1], dn = gate[2];
    const int64_t d = static_cast<int64_t>(col_block) * 256 + tid;
    if (d < D) {
        const float* br = basis + (b * D + d) * M;
        float* nbr = next_basis + (b * D + d) * M;
        float v = tanhf(to_f32(row[value_off + d]));
        if (novelty != nullptr) v = refine_value(v, fast[b * D + d]);
        float num = 0.0f;
        if (M == MAXM && reinterpret_cast<uintptr_t>(br) % 16 == 0 && reinterpret_cast<uintptr_t>(nbr) % 16 == 0) {
            // the whole basis row at once: MAXM / 4 16-byte loads in flight, then the stores
            float4 x4[MAXM / 4];
#pragma unroll
            for (int j = 0; j < MAXM / 4; ++j) x4[j] = reinterpret_cast<const float4*>(br)[j];
#pragma unroll
            for (int j = 0; j < MAXM / 4; ++j) {
                const float x[4] = {x4[j].x, x4[j].y, x4[j].z, x4[j].w};
                float o[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int m = 4 * j + c;
                    num = fmaf(x[c], q_sh[m], num);
                    o[c] = fmaf(decay, x[c], w * v * f_sh[m]);
                }
                reinterpret_cast<float4*>(nbr)[j] = make_float4(o[0], o[1], o[2], o[3]);
            }
        } else {
#pragma unroll
            for (int m = 0; m < MAXM; ++m) {
                if (m < M) {
                    const float x = br[m];
                    num = fmaf(x, q_sh[m], num);
                    nbr[m] = fmaf(decay, x, w * v * f_sh[m]);
                }
            }
        }
        const float reg = dn + kReadEpsilon;
        out[b * D + d] = (dn / reg) * num / reg;
    }
    if (col_block == 0 && tid < M) next_normalizer[b * M + tid] = fmaf(decay, normalizer[b * M + tid], w * f_sh[tid]);
}

}  // namespace step
}  // namespace koemi
