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
// small part); the three products of the window run on fp32 MFMA
// (v_mfma_f32_32x32x2f32): the feature similarities of the causal influence
// rows (K = features), the read itself (influence x values, K = slots, with
// the carried basis term as a few more K values) and, in the workgroups of the
// first row tile, the final basis columns (K = slots); the denominators and
// the normalizer are wave reductions.
#include "common.hpp"

namespace koemi {
namespace {

constexpr int kAssocCols = 64;     // output columns per workgroup
constexpr int kAssocRows = 64;     // query rows of one influence tile
constexpr float kMinDecay = 0.000244140625f;        // 2^-12
constexpr float kDecaySpan = 1.0f - 0.00048828125f;  // (1 - 2^-12) - 2^-12
constexpr float kReadEpsilon = 0.00390625f;          // 2^-8

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// LDS floats: the influence rows of the tile (64 x (Lq + 1), Lq = L rounded up
// to 32, the odd pitch spreading the MFMA operand reads of 32 rows over the
// banks); cum, log-decay (then the prior log-weights), write weights and
// final-write weights (4 Lq); features ([MAXM][L + 1]) and query features
// ([L][MAXM + 1]), zero-padded to MAXM so the feature products run unguarded;
// the value columns ([Lq][65]).
inline int64_t assoc_round(int64_t L) { return (L + 31) & ~int64_t(31); }
inline int64_t assoc_maxm(int64_t M) { return M <= 16 ? 16 : 32; }
inline size_t assoc_lds(int64_t L, int64_t M) {
    const int64_t Lq = assoc_round(L), X = assoc_maxm(M);
    return (kAssocRows * (Lq + 1) + 4 * Lq + X * (L + 1) + L * (X + 1) + Lq * (kAssocCols + 1)) * sizeof(float);
}

// e^x and tanh on the hardware exp2 and reciprocal (about 1 ulp each): the
// window kernel evaluates them per (query, slot) pair and per staged value.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float fast_tanh(float x) {
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(x * 2.8853900817779268f) + 1.0f);
}

// v_mfma_f32_32x32x2f32: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32];
// accumulator entry i of lane l is D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].
__device__ __forceinline__ f32x16 mfma2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// What one launch of assoc_read_kernel computes: the window's reads and its
// final state (kFull); only the final state's window terms with a zero
// carried state, sum_s e^{c_{L-1} - c_s} weight_s value_s features_s^T (and
// for the normalizer), plus e^{c_{L-1}} per row in `out` (kDelta; launched
// with one row tile); or only the reads (kRead).
constexpr int kFull = 0, kDelta = 1, kRead = 2;

template <int MAXM, int MODE = kFull>
__global__ __launch_bounds__(256) void assoc_read_kernel(
    const float* __restrict__ proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
    int64_t decay_off, int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ out,
    float* __restrict__ next_basis, float* __restrict__ next_normalizer, int L, int64_t D, int M) {
    extern __shared__ float sh[];
    constexpr int QP = MAXM + 1;        // query-feature pitch
    constexpr int VP = kAssocCols + 1;  // value pitch
    const int Lq = (L + 31) & ~31;
    const int IP = Lq + 1;  // influence pitch
    const int FP = L + 1;   // feature pitch
    float* infl = sh;                      // [64][IP]
    float* cum = infl + kAssocRows * IP;   // [Lq]
    float* logd = cum + Lq;                // [Lq]
    float* wt = logd + Lq;                 // [Lq] write weights
    float* fwt = wt + Lq;                  // [Lq] final-write weights
    float* f_sh = fwt + Lq;                // [MAXM][FP]
    float* q_sh = f_sh + MAXM * FP;        // [L][QP]
    float* val = q_sh + L * QP;            // [Lq][VP]
    const int64_t b = blockIdx.x;
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kAssocCols;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int h = lane >> 5, r32 = lane & 31;
    const float* rows0 = proj + b * L * stride;
    // the key's and the query's feature softmax of every position (one per
    // thread), the decay and the write weight with the key's
    for (int job = tid; job < 2 * L; job += 256) {
        const bool query = job >= L;
        const int t = query ? job - L : job;
        const float* row = rows0 + t * stride;
        const int64_t off = query ? fq_off : fk_off;
        float z[MAXM];
        float mx = -INFINITY;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) z[m] = row[off + min(m, M - 1)];  // unconditional, then masked
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            if (m >= M) z[m] = -INFINITY;
            mx = fmaxf(mx, z[m]);
        }
        float sum = 0.0f;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
            z[m] = m < M ? fast_exp(z[m] - mx) : 0.0f;
            sum += z[m];
        }
        const float inv = __builtin_amdgcn_rcpf(sum);
        if (query) {
#pragma unroll
            for (int m = 0; m < MAXM; ++m) q_sh[t * QP + m] = z[m] * inv;  // zero past M
        } else {
#pragma unroll
            for (int m = 0; m < MAXM; ++m) f_sh[m * FP + t] = z[m] * inv;
            const bool ok = valid[b * L + t] != 0;
            const float decay = kMinDecay + kDecaySpan * sigmoid_f(row[decay_off]);
            const float sv = fminf(fmaxf(surprise[b * L + t], 0.0f), 1.0f);
            logd[t] = ok ? logf(decay) : 0.0f;
            wt[t] = ok ? sigmoid_f(row[write_off]) * (0.25f + 0.75f * sv) : 0.0f;
        }
    }
    {
        // value rows t < Lq (zero past L): wave w stages rows w, w + 4, ...,
        // sixteen unconditional loads in flight per lane
        const int64_t dv = c0 + lane;
        const int64_t dc = dv < D ? dv : D - 1;
        for (int tb = wave; tb < Lq; tb += 64) {
            float x[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) x[j] = rows0[min(tb + 4 * j, L - 1) * stride + value_off + dc];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int t = tb + 4 * j;
                if (t < Lq) val[t * VP + lane] = (t < L && dv < D) ? fast_tanh(x[j]) : 0.0f;
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
    float* prior = logd;  // prior_t = cum_t - log decay_t replaces the log-decays from here on
    for (int s = tid; s < L; s += 256) {
        fwt[s] = expf(total - cum[s]) * wt[s];
        prior[s] = cum[s] - logd[s];
    }
    __syncthreads();

    if constexpr (MODE != kDelta) {
    const int t0 = static_cast<int>(blockIdx.z) * kAssocRows;
    const int rows = min(kAssocRows, L - t0);
    const int s_cnt = t0 + rows;  // slots that can reach these queries (s < t <= t0 + rows - 1)
    const int nsb = (s_cnt + 31) / 32;
    // influence of slot s on query t (zero unless s < t): the feature products
    // q_t . f_s of 32 x 32 blocks on MFMA (K = MAXM), then the decay and write
    // weights; blocks (query half, slot block) go round-robin over the waves.
    for (int blk = wave; blk < 2 * nsb; blk += 4) {
        const int tb = blk / nsb, sb = blk - tb * nsb;
        const int ta = min(t0 + tb * 32 + r32, L - 1);
        const int s = sb * 32 + r32, sc = min(s, L - 1);
        f32x16 acc = {};
#pragma unroll
        for (int kk = 0; kk < MAXM / 2; ++kk)
            acc = mfma2(q_sh[ta * QP + 2 * kk + h], f_sh[(2 * kk + h) * FP + sc], acc);
        const float cs = cum[sc], ws = wt[sc];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = tb * 32 + 8 * (i / 4) + 4 * h + (i % 4);
            const int t = t0 + r;
            const float v = fast_exp(prior[min(t, L - 1)] - cs) * acc[i] * ws;
            infl[r * IP + s] = (s < t && t < L) ? v : 0.0f;
        }
    }
    __syncthreads();
    {
        // the reads: wave w owns the 32 x 32 block (query half w / 2, column half w % 2);
        // sum over slots of influence x value on MFMA, then the carried basis term
        // e^{prior_t} (q_t . basis_d) as MAXM more K values. The denominators ride
        // along as a second product with the same A operand and B = 1 (row sums of
        // the influence), then e^{prior_t} (q_t . normalizer), so every lane holds
        // the denominator of each of its rows.
        const int tb = wave >> 1, db = wave & 1;
        const int k_end = (s_cnt + 1) & ~1;
        const float* ia = infl + (tb * 32 + r32) * IP + h;
        const float* vb = val + h * VP + db * 32 + r32;
        f32x16 acc = {}, accd = {};
        int s = 0;
        for (; s + 8 <= k_end; s += 8) {  // four steps' operands loaded together
            const float a0 = ia[s], a1 = ia[s + 2], a2 = ia[s + 4], a3 = ia[s + 6];
            const float b0 = vb[s * VP], b1 = vb[(s + 2) * VP], b2 = vb[(s + 4) * VP], b3 = vb[(s + 6) * VP];
            acc = mfma2(a0, b0, acc);
            accd = mfma2(a0, 1.0f, accd);
            acc = mfma2(a1, b1, acc);
            accd = mfma2(a1, 1.0f, accd);
            acc = mfma2(a2, b2, acc);
            accd = mfma2(a2, 1.0f, accd);
            acc = mfma2(a3, b3, acc);
            accd = mfma2(a3, 1.0f, accd);
        }
        for (; s < k_end; s += 2) {
            const float a = ia[s];
            acc = mfma2(a, vb[s * VP], acc);
            accd = mfma2(a, 1.0f, accd);
        }
        const int tq = min(t0 + tb * 32 + r32, L - 1);
        const float ep = fast_exp(prior[tq]);
        const int64_t dq = min(c0 + db * 32 + r32, D - 1);
#pragma unroll
        for (int kk = 0; kk < MAXM / 2; ++kk) {
            const int m = 2 * kk + h;
            const float on = m < M ? 1.0f : 0.0f;
            const float aq = ep * q_sh[tq * QP + m];
            acc = mfma2(aq, basis[(b * D + dq) * M + min(m, M - 1)] * on, acc);
            accd = mfma2(aq, normalizer[b * M + min(m, M - 1)] * on, accd);
        }
        const int64_t d = c0 + db * 32 + r32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = tb * 32 + 8 * (i / 4) + 4 * h + (i % 4);
            if (r >= rows || d >= D) continue;
            const float dn = accd[i], reg = dn + kReadEpsilon;
            out[(b * L + t0 + r) * D + d] = (dn / reg) * acc[i] / reg;
        }
    }
    }  // MODE != kDelta
    if constexpr (MODE == kRead) return;
    if (blockIdx.z != 0) return;
    // final basis columns (64 x M): sum over slots of (final-write weight x value)
    // x feature on MFMA, slots split in two halves over wave pairs, the halves
    // added through LDS (the influence rows are no longer read)
    const float keep = expf(total);
    const int half = ((L + 1) / 2 + 1) & ~1;
    {
        const int db = wave & 1, kh = wave >> 1;
        const int s_lo = kh * half, s_hi = min(L, s_lo + half);
        f32x16 acc = {};
        const float* fm = f_sh + min(r32, MAXM - 1) * FP;
        const float fon = r32 < MAXM ? 1.0f : 0.0f;
        const float* vcol = val + db * 32 + r32;
        for (int s = s_lo; s < s_hi; s += 8) {  // four steps' operands loaded together
            float a[4], bf[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int sl = s + 2 * q + h, slc = min(sl, L - 1);
                a[q] = sl < s_hi ? fwt[slc] * vcol[slc * VP] : 0.0f;
                bf[q] = fm[slc] * fon;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = mfma2(a[q], bf[q], acc);
        }
        __syncthreads();  // the influence area is free
        float* part = infl + db * 16 * kWave;  // [2][16][64]
        if (kh == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) part[i * kWave + lane] = acc[i];
        }
        __syncthreads();
        if (kh == 0) {
            const int m = r32;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t d = c0 + db * 32 + 8 * (i / 4) + 4 * h + (i % 4);
                if (m >= M || d >= D) continue;
                const int64_t at = (b * D + d) * M + m;
                const float window_terms = acc[i] + part[i * kWave + lane];
                next_basis[at] = MODE == kDelta ? window_terms : fmaf(keep, basis[at], window_terms);
            }
        }
    }
    if (blockIdx.y == 0 && wave == 3) {
        for (int m = 0; m < M; ++m) {
            float sum = 0.0f;
            for (int s = lane; s < L; s += kWave) sum = fmaf(fwt[s], f_sh[m * FP + s], sum);
            sum = wave_sum_xor(sum);
            if (lane == 0) next_normalizer[b * M + m] = MODE == kDelta ? sum : fmaf(keep, normalizer[b * M + m], sum);
        }
        if (MODE == kDelta && lane == 0) out[b] = keep;
    }
}

// The state carried into each of a sequence's windows and the state after the
// last: for element e of the flattened basis (D x M, then the M normalizer
// entries) of batch row b, cur = state_0; window w receives cur, then
// cur = fmaf(keep_w, cur, delta_w), the update assoc_read_kernel applies at the
// end of a window (so the carried states equal a window-by-window run's).
__global__ __launch_bounds__(256) void assoc_carry_kernel(
    const float* __restrict__ delta_basis, const float* __restrict__ delta_norm, const float* __restrict__ keep,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ carried_basis,
    float* __restrict__ carried_norm, float* __restrict__ next_basis, float* __restrict__ next_normalizer,
    int64_t windows, int64_t DM, int64_t M) {
    const int64_t b = blockIdx.x;
    const int64_t e = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x;
    if (e >= DM + M) return;
    const bool is_basis = e < DM;
    const int64_t x = is_basis ? e : e - DM;
    const int64_t n = is_basis ? DM : M;
    const float* delta = is_basis ? delta_basis : delta_norm;
    float* carried = is_basis ? carried_basis : carried_norm;
    float cur = is_basis ? basis[b * DM + x] : normalizer[b * M + x];
    for (int64_t w = 0; w < windows; ++w) {
        const int64_t row = b * windows + w;
        carried[row * n + x] = cur;
        cur = fmaf(keep[row], cur, delta[row * n + x]);
    }
    (is_basis ? next_basis : next_normalizer)[b * n + x] = cur;
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
    if (tid < kWave) {
        // lanes 0..31: the key's feature softmax, lanes 32..63: the query's
        // (one feature per lane; max and sum by shuffles within each half)
        const int lane = tid, m = lane & 31;
        const bool query = lane >= 32, in = m < M;
        const float z = in ? row[(query ? fq_off : fk_off) + min(m, M - 1)] : -INFINITY;
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
            gate[0] = ok ? kMinDecay + kDecaySpan * sigmoid_f(row[decay_off]) : 1.0f;
            gate[1] = ok ? sigmoid_f(row[write_off]) * (0.25f + 0.75f * sv) : 0.0f;
        }
    }
    __syncthreads();
    const float decay = gate[0], w = gate[1], dn = gate[2];
    const int64_t d = static_cast<int64_t>(blockIdx.y) * 256 + tid;
    if (d < D) {
        const float* br = basis + (b * D + d) * M;
        float* nbr = next_basis + (b * D + d) * M;
        const float v = tanhf(row[value_off + d]);
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

namespace {

struct WindowsWorkspace {
    size_t delta_basis, delta_norm, keep, carried_basis, carried_norm, total;
};

inline size_t align256w(size_t x) { return (x + 255) & ~size_t(255); }

inline WindowsWorkspace windows_workspace(int64_t rows, int64_t width, int64_t features) {
    WindowsWorkspace w;
    const size_t basis_bytes = align256w(static_cast<size_t>(rows * width * features) * sizeof(float));
    const size_t norm_bytes = align256w(static_cast<size_t>(rows * features) * sizeof(float));
    w.delta_basis = 0;
    w.delta_norm = w.delta_basis + basis_bytes;
    w.keep = w.delta_norm + norm_bytes;
    w.carried_basis = w.keep + align256w(static_cast<size_t>(rows) * sizeof(float));
    w.carried_norm = w.carried_basis + basis_bytes;
    w.total = w.carried_norm + norm_bytes;
    return w;
}

}  // namespace

extern "C" size_t koemi_assoc_scan_read_windows_workspace_bytes(int64_t batch, int64_t windows, int64_t width,
                                                                 int64_t features) {
    if (batch < 0 || windows < 0 || width < 1 || features < 1) return 0;
    return windows_workspace(batch * windows, width, features).total;
}

extern "C" int koemi_assoc_scan_read_windows(const float* projections, int64_t row_stride, int64_t value_offset,
                                             int64_t feature_offset, int64_t query_feature_offset,
                                             int64_t decay_offset, int64_t write_offset, const float* surprise,
                                             const uint8_t* valid, const float* basis, const float* normalizer,
                                             float* read, float* next_basis, float* next_normalizer, int64_t batch,
                                             int64_t windows, int64_t window, int64_t width, int64_t features,
                                             void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || windows < 0 || window < 2 || width < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "windowed associative read needs non-negative batch and windows, a window of at "
                    "least two positions, positive width and features");
    if (features > 32) return fail(KOEMI_ERR_UNSUPPORTED, "associative read supports at most 32 memory features");
    auto inside = [&](int64_t off, int64_t span) { return off >= 0 && off + span <= row_stride; };
    if (!inside(value_offset, width) || !inside(feature_offset, features) ||
        !inside(query_feature_offset, features) || !inside(decay_offset, 1) || !inside(write_offset, 1))
        return fail(KOEMI_ERR_INVALID, "associative read column offsets must lie inside the row stride");
    const int64_t rows = batch * windows;
    if (batch == 0) return KOEMI_OK;
    const size_t lds = assoc_lds(window, features);
    if (lds > 160 * 1024)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read window too long (%lld positions)",
                    static_cast<long long>(window));
    if (rows > 0x7fffffffLL || (width + kAssocCols - 1) / kAssocCols > 65535 ||
        (width * features + features + 255) / 256 > 65535)
        return fail(KOEMI_ERR_UNSUPPORTED, "windowed associative read grid too large");
    if (!basis || !normalizer || !next_basis || !next_normalizer ||
        (windows > 0 && (!projections || !surprise || !valid || !read)))
        return fail(KOEMI_ERR_INVALID, "windowed associative read received a null pointer");
    const WindowsWorkspace ws = windows_workspace(rows, width, features);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "windowed associative read workspace too small: need %zu bytes", ws.total);
    char* w = static_cast<char*>(workspace);
    float* delta_basis = reinterpret_cast<float*>(w + ws.delta_basis);
    float* delta_norm = reinterpret_cast<float*>(w + ws.delta_norm);
    float* keep = reinterpret_cast<float*>(w + ws.keep);
    float* carried_basis = reinterpret_cast<float*>(w + ws.carried_basis);
    float* carried_norm = reinterpret_cast<float*>(w + ws.carried_norm);
    const hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(features);
    const unsigned col_tiles = static_cast<unsigned>((width + kAssocCols - 1) / kAssocCols);
    auto launch = [&](auto kernel, unsigned row_tiles, const float* carried_b, const float* carried_n, float* out,
                      float* nb, float* nn) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(rows), col_tiles, row_tiles), dim3(256), lds, s,
                           projections, row_stride, value_offset, feature_offset, query_feature_offset, decay_offset,
                           write_offset, surprise, valid, carried_b, carried_n, out, nb, nn, static_cast<int>(window),
                           width, M);
    };
    if (windows > 0) {
        // 1. every window's own terms of the final state, from a zero carried state
        if (M <= 16) launch(assoc_read_kernel<16, kDelta>, 1u, nullptr, nullptr, keep, delta_basis, delta_norm);
        else launch(assoc_read_kernel<32, kDelta>, 1u, nullptr, nullptr, keep, delta_basis, delta_norm);
        int st = check_launch("koemi_assoc_scan_read_windows(delta)");
        if (st != KOEMI_OK) return st;
    }
    // 2. the state carried into each window, and the final state
    const int64_t DM = width * features;
    hipLaunchKernelGGL(assoc_carry_kernel, dim3(static_cast<unsigned>(batch), static_cast<unsigned>((DM + M + 255) / 256)),
                       dim3(256), 0, s, delta_basis, delta_norm, keep, basis, normalizer, carried_basis, carried_norm,
                       next_basis, next_normalizer, windows, DM, static_cast<int64_t>(M));
    int st = check_launch("koemi_assoc_scan_read_windows(carry)");
    if (st != KOEMI_OK || windows == 0) return st;
    // 3. the reads of every window from its carried state
    const unsigned row_tiles = static_cast<unsigned>((window + kAssocRows - 1) / kAssocRows);
    if (M <= 16) launch(assoc_read_kernel<16, kRead>, row_tiles, carried_basis, carried_norm, read, nullptr, nullptr);
    else launch(assoc_read_kernel<32, kRead>, row_tiles, carried_basis, carried_norm, read, nullptr, nullptr);
    return check_launch("koemi_assoc_scan_read_windows(read)");
}
