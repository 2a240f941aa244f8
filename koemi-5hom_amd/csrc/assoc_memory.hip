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
// Windows of one position (a decode step) take assoc_step_kernel: the read
// from the carried state, then the state update (memory.py:91-95, 279-288),
// one thread per (batch row, column). Longer windows take assoc_read_kernel,
// one workgroup per (batch row, 64 output columns, 64 query rows): the
// window's feature softmaxes, decays, cumulative log-decays and write weights
// are formed while staging them in LDS (each workgroup of a row repeats this
// small part), then the causal influence rows of its 64 queries go to LDS
// with their sums (wave reductions), and four waves of 16 rows each
// accumulate the read of their 64 columns, four slots per LDS load; the
// workgroups of the first row tile also write the final basis columns and the
// normalizer.
#include "common.hpp"

namespace koemi {
namespace {

constexpr int kAssocCols = 64;     // output columns per workgroup
constexpr int kAssocRows = 64;     // query rows of one influence tile
constexpr float kMinDecay = 0.000244140625f;        // 2^-12
constexpr float kDecaySpan = 1.0f - 0.00048828125f;  // (1 - 2^-12) - 2^-12
constexpr float kReadEpsilon = 0.00390625f;          // 2^-8

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// LDS floats: the influence rows of the tile (64 x L rounded up to 4, for
// 16-byte reads) and their denominators (64), cum, log-decay, write weights
// and final-write weights (4L), features (transposed, [MAXM][L]) and query
// features ([L][MAXM]) zero-padded to MAXM so every feature loop runs
// unguarded (2 L MAXM), the value columns (64L).
inline int64_t assoc_pitch(int64_t L) { return (L + 3) & ~int64_t(3); }
inline int64_t assoc_maxm(int64_t M) { return M <= 16 ? 16 : 32; }
inline size_t assoc_lds(int64_t L, int64_t M) {
    return (kAssocRows * assoc_pitch(L) + kAssocRows + 4 * L + 2 * L * assoc_maxm(M) + kAssocCols * L) * sizeof(float);
}

template <int MAXM>
__global__ __launch_bounds__(256) void assoc_read_kernel(
    const float* __restrict__ proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
    int64_t decay_off, int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ out,
    float* __restrict__ next_basis, float* __restrict__ next_normalizer, int L, int64_t D, int M) {
    extern __shared__ float sh[];
    const int Lp = (L + 3) & ~3;
    float* infl = sh;                     // [64][Lp]
    float* den = infl + kAssocRows * Lp;  // [64]
    float* cum = den + kAssocRows;        // [L]
    float* logd = cum + L;                // [L]
    float* wt = logd + L;                 // [L] write weights
    float* fwt = wt + L;                  // [L] final-write weights
    float* f_sh = fwt + L;                // [MAXM][L] (slot-contiguous: lanes read consecutive slots)
    float* q_sh = f_sh + L * MAXM;        // [L][MAXM]
    float* val = q_sh + L * MAXM;         // [L][64]
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
        for (int m = 0; m < MAXM; ++m) {  // unconditional loads at clamped columns, then masked
            zk[m] = row[fk_off + min(m, M - 1)];
            zq[m] = row[fq_off + min(m, M - 1)];
        }
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            if (m >= M) zk[m] = zq[m] = -INFINITY;
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
            f_sh[m * L + t] = zk[m] / sk;  // zero past M
            q_sh[t * MAXM + m] = zq[m] / sq;
        }
        const bool ok = valid[b * L + t] != 0;
        const float decay = kMinDecay + kDecaySpan * sigmoid_f(row[decay_off]);
        const float sv = fminf(fmaxf(surprise[b * L + t], 0.0f), 1.0f);
        logd[t] = ok ? logf(decay) : 0.0f;
        wt[t] = ok ? sigmoid_f(row[write_off]) * (0.25f + 0.75f * sv) : 0.0f;
    }
    {
        // wave w stages value rows w, w + 4, ...: eight loads in flight per lane per batch
        const int64_t dv = c0 + lane;
        for (int tb = wave; tb < L; tb += 32) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int t = tb + 4 * j;
                x[j] = (t < L && dv < D) ? rows0[t * stride + value_off + dv] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int t = tb + 4 * j;
                if (t < L) val[t * kAssocCols + lane] = dv < D ? tanhf(x[j]) : 0.0f;
            }
        }
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
    const int t0 = static_cast<int>(blockIdx.z) * kAssocRows;
    const int rows = min(kAssocRows, L - t0);
    __syncthreads();  // fwt is written
    // influence of slot s on query t0 + r (zero unless s < t): wave w fills
    // rows w, w + 4, ...; lanes take consecutive slots; the row sums (the
    // reads' denominators) by wave reduction.
    for (int r = wave; r < rows; r += 4) {
        const int t = t0 + r;
        const float prior = cum[t] - logd[t];
        float sum = 0.0f;
        for (int s = lane; s < t0 + rows; s += kWave) {
            float v = 0.0f;
            if (s < t) {
                float sim = 0.0f;
#pragma unroll
                for (int m = 0; m < MAXM; ++m) sim = fmaf(q_sh[t * MAXM + m], f_sh[m * L + s], sim);
                v = expf(prior - cum[s]) * sim * wt[s];
            }
            infl[r * Lp + s] = v;
            sum += v;
        }
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
        if (lane == 0) {
            float nq = 0.0f;
#pragma unroll
            for (int m = 0; m < MAXM; ++m) nq = fmaf(nrm[m], q_sh[t * MAXM + m], nq);
            den[r] = expf(prior) * nq + sum;
        }
    }
    __syncthreads();
    // wave w: rows w, w + 4, ... of the tile (16 at most), lane = column
    float acc[kRowsPerWave];
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) acc[j] = 0.0f;
    const int s_end = t0 + rows - 1;  // slots past the tile's last query add zero
    int s = 0;
    if (rows == kAssocRows) {
        for (; s + 4 <= s_end; s += 4) {
            const float v0 = val[s * kAssocCols + lane], v1 = val[(s + 1) * kAssocCols + lane];
            const float v2 = val[(s + 2) * kAssocCols + lane], v3 = val[(s + 3) * kAssocCols + lane];
#pragma unroll
            for (int j = 0; j < kRowsPerWave; ++j) {
                const float4 iv = *reinterpret_cast<const float4*>(infl + (wave + 4 * j) * Lp + s);
                acc[j] = fmaf(iv.x, v0, fmaf(iv.y, v1, fmaf(iv.z, v2, fmaf(iv.w, v3, acc[j]))));
            }
        }
    }
    for (; s < s_end; ++s) {
        const float v0 = val[s * kAssocCols + lane];
#pragma unroll
        for (int j = 0; j < kRowsPerWave; ++j) {
            const int r = wave + 4 * j;
            if (r < rows) acc[j] = fmaf(infl[r * Lp + s], v0, acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kRowsPerWave; ++j) {
        const int r = wave + 4 * j;
        if (r >= rows) continue;
        const int t = t0 + r;
        float bq = 0.0f;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) bq = fmaf(brow[m], q_sh[t * MAXM + m], bq);
        const float num = expf(cum[t] - logd[t]) * bq + acc[j];
        const float dn = den[r], reg = dn + kReadEpsilon;
        if (dok) out[(b * L + t) * D + d] = (dn / reg) * num / reg;
    }
    if (blockIdx.z != 0) return;
    // final basis columns: wave w takes the features m with m % 4 == w
    const float keep = expf(total);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
        if (m >= M || (m & 3) != wave) continue;
        float a0 = keep * brow[m], a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        int s = 0;
        for (; s + 4 <= L; s += 4) {
            a0 = fmaf(fwt[s] * val[s * kAssocCols + lane], f_sh[m * L + s], a0);
            a1 = fmaf(fwt[s + 1] * val[(s + 1) * kAssocCols + lane], f_sh[m * L + s + 1], a1);
            a2 = fmaf(fwt[s + 2] * val[(s + 2) * kAssocCols + lane], f_sh[m * L + s + 2], a2);
            a3 = fmaf(fwt[s + 3] * val[(s + 3) * kAssocCols + lane], f_sh[m * L + s + 3], a3);
        }
        for (; s < L; ++s) a0 = fmaf(fwt[s] * val[s * kAssocCols + lane], f_sh[m * L + s], a0);
        if (dok) next_basis[(b * D + d) * M + m] = (a0 + a1) + (a2 + a3);
    }
    if (blockIdx.y == 0 && tid < M) {
        float acc = keep * normalizer[b * M + tid];
        for (int s = 0; s < L; ++s) acc = fmaf(fwt[s], f_sh[tid * L + s], acc);
        next_normalizer[b * M + tid] = acc;
    }
}

// One-position window (a decode step): read from the carried state, then
// basis' = decay basis + weight value features^T, normalizer' likewise.
// One thread per (batch row, column); the row's softmaxes and gates in LDS.
template <int MAXM>
__global__ __launch_bounds__(256) void assoc_step_kernel(
    const float* __restrict__ proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
    int64_t decay_off, int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ out,
    float* __restrict__ next_basis, float* __restrict__ next_normalizer, int64_t D, int M) {
    __shared__ float f_sh[MAXM], q_sh[MAXM], gate[3];  // decay, weight, normalizer . query features
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x;
    const float* row = proj + b * stride;
    if (tid == 0) {
        float zk[MAXM], zq[MAXM], mk = -INFINITY, mq = -INFINITY;
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
        float nq = 0.0f;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            f_sh[m] = zk[m] / sk;
            q_sh[m] = zq[m] / sq;
            if (m < M) nq = fmaf(normalizer[b * M + m], q_sh[m], nq);
        }
        const bool ok = valid[b] != 0;
        const float sv = fminf(fmaxf(surprise[b], 0.0f), 1.0f);
        gate[0] = ok ? kMinDecay + kDecaySpan * sigmoid_f(row[decay_off]) : 1.0f;
        gate[1] = ok ? sigmoid_f(row[write_off]) * (0.25f + 0.75f * sv) : 0.0f;
        gate[2] = nq;
    }
    __syncthreads();
    const float decay = gate[0], w = gate[1], dn = gate[2];
    const int64_t d = static_cast<int64_t>(blockIdx.y) * 256 + tid;
    if (d < D) {
        const float* br = basis + (b * D + d) * M;
        float* nbr = next_basis + (b * D + d) * M;
        const float v = tanhf(row[value_off + d]);
        float num = 0.0f;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            if (m < M) {
                const float x = br[m];
                num = fmaf(x, q_sh[m], num);
                nbr[m] = fmaf(decay, x, w * v * f_sh[m]);
            }
        }
        const float reg = dn + kReadEpsilon;
        out[b * D + d] = (dn / reg) * num / reg;
    }
    if (blockIdx.y == 0 && tid < M) next_normalizer[b * M + tid] = fmaf(decay, normalizer[b * M + tid], w * f_sh[tid]);
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
    if (length == 1) {
        const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((width + 255) / 256));
        auto step = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, projections, row_stride, value_offset, feature_offset,
                               query_feature_offset, decay_offset, write_offset, surprise, valid, basis, normalizer,
                               read, next_basis, next_normalizer, width, M);
        };
        if (M <= 16) step(assoc_step_kernel<16>);
        else step(assoc_step_kernel<32>);
        return check_launch("koemi_assoc_scan_read");
    }
    const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((width + kAssocCols - 1) / kAssocCols),
                    static_cast<unsigned>((length + kAssocRows - 1) / kAssocRows));
    auto run = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), lds, s, projections, row_stride, value_offset, feature_offset,
                           query_feature_offset, decay_offset, write_offset, surprise, valid, basis, normalizer, read,
                           next_basis, next_normalizer, static_cast<int>(length), width, M);
    };
    if (M <= 16) run(assoc_read_kernel<16>);
    else run(assoc_read_kernel<32>);
    return check_launch("koemi_assoc_scan_read");
}
