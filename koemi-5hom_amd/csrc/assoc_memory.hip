// Associative (fast-weight) memory of the HERM block window for gfx950.
//
// Reference: HierarchicalAssociativeMemory.project, query_features,
// fast_write_terms and scan_and_read (model/memory.py:82-144, 244-255) with
// the write masking of network.py:734-740, all torch composites in the
// reference. Per batch row, over the window's positions t < L:
//
//   features_t = softmax(W_f key_t + b_f)          query_t' = softmax(W_f query_t + b_f)
//   value_t    = tanh(v_t)                         decay_t  = 2^-12 + (1 - 2^-11) sigmoid(d_t)
//   weight_t   = sigmoid(w_t) (0.25 + 0.75 clamp(surprise_t, 0, 1))
//   invalid t: decay 1, weight 0
//   c_t = sum_{s<=t} log decay_s,  prior_t = c_t - log decay_t
//   num_t = e^{prior_t} (basis query_t') + sum_{s<t} e^{prior_t - c_s} (features_s . query_t') weight_s value_s
//   den_t = e^{prior_t} (normalizer . query_t') + sum_{s<t} (the same coefficients)
//   read_t = den/(den + 2^-8) * num/(den + 2^-8)
//   basis'  = e^{c_{L-1}} basis + sum_s e^{c_{L-1} - c_s} weight_s value_s features_s^T, normalizer' likewise.
//
// The caller's stacked projection of the working states supplies, as columns
// of one fp32 matrix addressed by row stride and column offsets, the value
// pre-activations v (width columns), the feature logits W_f key + b_f and
// W_f query + b_f (M columns each: key and query are linear in the states, so
// W_f W_k and W_f W_q fold into that projection) and the decay and write
// logits (one column each).
//
// One kernel, one workgroup per (batch row, 64 output columns): the window's
// feature softmaxes, decays, cumulative log-decays and write weights are
// formed while staging them in LDS (each workgroup of a row repeats this small
// part), then the causal influence matrix of 64 query rows at a time goes to
// LDS and four waves of 16 rows each accumulate the read of their 64 columns,
// four slots per LDS load; the final basis columns and the normalizer come
// from the same LDS data.
#include "common.hpp"

namespace koemi {
namespace {

constexpr int kAssocCols = 64;     // output columns per workgroup
constexpr int kAssocRows = 64;     // query rows of one influence tile
constexpr float kMinDecay = 0.000244140625f;        // 2^-12
constexpr float kDecaySpan = 1.0f - 0.00048828125f;  // (1 - 2^-12) - 2^-12
constexpr float kReadEpsilon = 0.00390625f;          // 2^-8

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// LDS floats: cum, log-decay, write weights and final-write weights (4L),
// features (transposed, [M][L]) and query features ([L][M]) (2LM), the value
// columns (64L) and one influence tile (64L).
inline size_t assoc_lds(int64_t L, int64_t M) { return (4 * L + 2 * L * M + 2 * kAssocCols * L) * sizeof(float); }

template <int MAXM>
__global__ __launch_bounds__(256) void assoc_read_kernel(
    const float* __restrict__ proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
    int64_t decay_off, int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ out,
    float* __restrict__ next_basis, float* __restrict__ next_normalizer, int L, int64_t D, int M) {
    extern __shared__ float sh[];
    float* cum = sh;                      // [L]
    float* logd = cum + L;                // [L]
    float* wt = logd + L;                 // [L] write weights
    float* fwt = wt + L;                  // [L] final-write weights
    float* f_sh = fwt + L;                // [M][L] (slot-contiguous: lanes read consecutive slots)
    float* q_sh = f_sh + L * M;           // [L][M]
    float* val = q_sh + L * M;            // [L][64]
    float* infl = val + L * kAssocCols;   // [64][L]
    const int64_t b = blockIdx.x;
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kAssocCols;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const float* rows0 = proj + b * L * stride;
    // per position: the two feature softmaxes, the decay and the write weight
    for (int t = tid; t < L; t += 256) {
        const float* row = rows0 + t * stride;
        float zk[MAXM], zq[MAXM];
        float mk = -INFINITY, mq = -INFINITY;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            zk[m] = m < M ? row[fk_off + m] : -INFINITY;
            zq[m] = m < M ? row[fq_off + m] : -INFINITY;
            mk = fmaxf(mk, zk[m]);
            mq = fmaxf(mq, zq[m]);
        }
        float sk = 0.0f, sq = 0.0f;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            zk[m] = m < M ? expf(zk[m] - mk) : 0.0f;
            zq[m] = m < M ? expf(zq[m] - mq) : 0.0f;
            sk += zk[m];
            sq += zq[m];
        }
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            if (m < M) {
                f_sh[m * L + t] = zk[m] / sk;
                q_sh[t * M + m] = zq[m] / sq;
            }
        }
        const bool ok = valid[b * L + t] != 0;
        const float decay = kMinDecay + kDecaySpan * sigmoid_f(row[decay_off]);
        const float sv = fminf(fmaxf(surprise[b * L + t], 0.0f), 1.0f);
        logd[t] = ok ? logf(decay) : 0.0f;
        wt[t] = ok ? sigmoid_f(row[write_off]) * (0.25f + 0.75f * sv) : 0.0f;
    }
    for (int t = wave; t < L; t += 4) {
        const int64_t d = c0 + lane;
        val[t * kAssocCols + lane] = d < D ? tanhf(rows0[t * stride + value_off + d]) : 0.0f;
    }
    __syncthreads();
    if (wave == 0) {
        // cumulative log-decay (memory.py:108): lane l sums its run of positions
        // [l R, l R + R); an inclusive wave scan of the run sums places it.
        const int R = (L + kWave - 1) / kWave;
        float acc = 0.0f;
        for (int j = 0; j < R; ++j) {
            const int t = lane * R + j;
            if (t < L) acc += logd[t];
        }
        float incl = acc;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const float up = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += up;
        }
        float c = incl - acc;
        for (int j = 0; j < R; ++j) {
            const int t = lane * R + j;
            if (t < L) {
                c += logd[t];
                cum[t] = c;
            }
        }
    }
    __syncthreads();
    const float total = cum[L - 1];
    for (int s = tid; s < L; s += 256) fwt[s] = expf(total - cum[s]) * wt[s];
    const int64_t d = c0 + lane;
    const bool dok = d < D;
    float brow[MAXM], nrm[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        brow[m] = (m < M && dok) ? basis[(b * D + d) * M + m] : 0.0f;
        nrm[m] = m < M ? normalizer[b * M + m] : 0.0f;
    }

    constexpr int kRowsPerWave = kAssocRows / 4;
    for (int t0 = 0; t0 < L; t0 += kAssocRows) {
        const int rows = min(kAssocRows, L - t0);
        __syncthreads();  // fwt is written; the previous tile's readers are done with infl
        // influence of slot s on query t0 + r (zero unless s < t): wave w fills
        // rows w, w + 4, ...; lanes take consecutive slots.
        for (int r = wave; r < rows; r += 4) {
            const int t = t0 + r;
            const float prior = cum[t] - logd[t];
            for (int s = lane; s < L; s += kWave) {
                float v = 0.0f;
                if (s < t) {
                    float sim = 0.0f;
                    for (int m = 0; m < M; ++m) sim = fmaf(q_sh[t * M + m], f_sh[m * L + s], sim);
                    v = expf(prior - cum[s]) * sim * wt[s];
                }
                infl[r * L + s] = v;
            }
        }
        __syncthreads();
        // wave w: rows w, w + 4, ... of the tile (16 at most), lane = column;
        // the row's denominator sum rides along (the same in every lane).
        float acc[kRowsPerWave], dsum[kRowsPerWave];
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) acc[j] = dsum[j] = 0.0f;
        const int s_end = t0 + rows - 1;  // slots past the tile's last query add zero
        int s = 0;
        for (; s + 4 <= s_end; s += 4) {
            const float v0 = val[s * kAssocCols + lane], v1 = val[(s + 1) * kAssocCols + lane];
            const float v2 = val[(s + 2) * kAssocCols + lane], v3 = val[(s + 3) * kAssocCols + lane];
#pragma unroll
            for (int j = 0; j < kRowsPerWave; ++j) {
                const int r = wave + 4 * j;
                if (r < rows) {
                    const float* ir = infl + r * L + s;
                    const float i0 = ir[0], i1 = ir[1], i2 = ir[2], i3 = ir[3];
                    acc[j] = fmaf(i0, v0, fmaf(i1, v1, fmaf(i2, v2, fmaf(i3, v3, acc[j]))));
                    dsum[j] += (i0 + i1) + (i2 + i3);
                }
            }
        }
        for (; s < s_end; ++s) {
            const float v0 = val[s * kAssocCols + lane];
#pragma unroll
            for (int j = 0; j < kRowsPerWave; ++j) {
                const int r = wave + 4 * j;
                if (r < rows) {
                    const float i0 = infl[r * L + s];
                    acc[j] = fmaf(i0, v0, acc[j]);
                    dsum[j] += i0;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int r = wave + 4 * j;
            if (r >= rows) continue;
            const int t = t0 + r;
            float bq = 0.0f, nq = 0.0f;
#pragma unroll
            for (int m = 0; m < MAXM; ++m) {
                if (m < M) {
                    bq = fmaf(brow[m], q_sh[t * M + m], bq);
                    nq = fmaf(nrm[m], q_sh[t * M + m], nq);
                }
            }
            const float initial = expf(cum[t] - logd[t]);
            const float num = initial * bq + acc[j];
            const float dn = initial * nq + dsum[j], reg = dn + kReadEpsilon;
            if (dok) out[(b * L + t) * D + d] = (dn / reg) * num / reg;
        }
    }
    // final basis columns: wave w takes the features m with m % 4 == w
    const float keep = expf(total);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        if (m >= M || (m & 3) != wave) continue;
        float acc = keep * brow[m];
        for (int s = 0; s < L; ++s) acc = fmaf(fwt[s] * val[s * kAssocCols + lane], f_sh[m * L + s], acc);
        if (dok) next_basis[(b * D + d) * M + m] = acc;
    }
    if (blockIdx.y == 0 && tid < M) {
        float acc = keep * normalizer[b * M + tid];
        for (int s = 0; s < L; ++s) acc = fmaf(fwt[s], f_sh[tid * L + s], acc);
        next_normalizer[b * M + tid] = acc;
    }
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_assoc_scan_read(const float* projections, int64_t row_stride, int64_t value_offset,
                                     int64_t feature_offset, int64_t query_feature_offset, int64_t decay_offset,
                                     int64_t write_offset, const float* surprise, const uint8_t* valid,
                                     const float* basis, const float* normalizer, float* read, float* next_basis,
                                     float* next_normalizer, int64_t batch, int64_t length, int64_t width,
                                     int64_t features, koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "associative read needs non-negative batch and length, positive width and features");
    if (features > 32) return fail(KOEMI_ERR_UNSUPPORTED, "associative read supports at most 32 memory features");
    auto inside = [&](int64_t off, int64_t span) { return off >= 0 && off + span <= row_stride; };
    if (!inside(value_offset, width) || !inside(feature_offset, features) ||
        !inside(query_feature_offset, features) || !inside(decay_offset, 1) || !inside(write_offset, 1))
        return fail(KOEMI_ERR_INVALID, "associative read column offsets must lie inside the row stride");
    if (batch == 0 || length == 0) return KOEMI_OK;
    const size_t lds = assoc_lds(length, features);
    if (lds > 160 * 1024)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read window too long (%lld positions)",
                    static_cast<long long>(length));
    if (batch > 0x7fffffffLL || (width + kAssocCols - 1) / kAssocCols > 65535)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read grid too large");
    if (!projections || !surprise || !valid || !basis || !normalizer || !read || !next_basis || !next_normalizer)
        return fail(KOEMI_ERR_INVALID, "associative read received a null pointer");
    const hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(features);
    const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((width + kAssocCols - 1) / kAssocCols));
    auto run = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), lds, s, projections, row_stride, value_offset, feature_offset,
                           query_feature_offset, decay_offset, write_offset, surprise, valid, basis, normalizer, read,
                           next_basis, next_normalizer, static_cast<int>(length), width, M);
    };
    if (M <= 16) run(assoc_read_kernel<16>);
    else run(assoc_read_kernel<32>);
    return check_launch("koemi_assoc_scan_read");
}
