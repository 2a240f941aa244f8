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
// one thread per (batch row, column). Longer windows take three launches:
// assoc_prep_kernel forms each row's feature softmaxes, decays, cumulative
// log-decays and write weights once, into a workspace; assoc_delta_kernel the
// window's own terms of the final state (fp32 MFMA, K = slots);
// assoc_window_read_kernel the reads: the causal influence rows of 64 queries
// (fp32 MFMA, K = features) in LDS, then influence x values plus the carried
// basis term on MFMA, the denominators as wave reductions. The projection may
// be fp32 or bf16 (the GEMM's own output dtype); everything after the load is
// fp32.
#include "common.hpp"
#include "step_memory.hpp"

#include <type_traits>

namespace koemi {
namespace {

constexpr int kAssocCols = 64;     // output columns per workgroup
constexpr int kAssocRows = 64;     // query rows of one influence tile
using step::kDecaySpan;
using step::kMinDecay;
using step::kReadEpsilon;
using step::sigmoid_f;

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// e^x and tanh on the hardware exp2 and reciprocal (about 1 ulp each): the
// window kernels evaluate them per (query, slot) pair and per value read.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
__device__ __forceinline__ float fast_tanh(float x) {
    return 1.0f - 2.0f * __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(x * 2.8853900817779268f) + 1.0f);
}

// v_mfma_f32_32x32x2f32: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32];
// accumulator entry i of lane l is D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].
__device__ __forceinline__ f32x16 mfma2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

inline int64_t assoc_maxm(int64_t M) { return M <= 16 ? 16 : 32; }

// Per-position quantities of a window row, formed once by assoc_prep_kernel
// and read by the delta and read kernels: the key's and the query's feature
// softmaxes ([rows][L][MAXM], zero past M), the cumulative log-decay c_t, the
// prior log-weight c_t - log decay_t, the write weight, the final-write weight
// e^{c_{L-1} - c_t} weight_t, and per row e^{c_{L-1}}.
struct AssocPrep {
    float* kf;
    float* qf;
    float* cum;
    float* prior;
    float* wt;
    float* fwt;
    float* keep;
};

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
inline size_t prep_bytes(int64_t rows, int64_t L, int64_t M) {
    const size_t feat = align256(static_cast<size_t>(rows * L * assoc_maxm(M)) * sizeof(float));
    const size_t pos = align256(static_cast<size_t>(rows * L) * sizeof(float));
    return 2 * feat + 4 * pos + align256(static_cast<size_t>(rows) * sizeof(float));
}
inline AssocPrep prep_at(void* base, int64_t rows, int64_t L, int64_t M) {
    char* w = static_cast<char*>(base);
    const size_t feat = align256(static_cast<size_t>(rows * L * assoc_maxm(M)) * sizeof(float));
    const size_t pos = align256(static_cast<size_t>(rows * L) * sizeof(float));
    AssocPrep p;
    p.kf = reinterpret_cast<float*>(w);
    p.qf = reinterpret_cast<float*>(w + feat);
    p.cum = reinterpret_cast<float*>(w + 2 * feat);
    p.prior = reinterpret_cast<float*>(w + 2 * feat + pos);
    p.wt = reinterpret_cast<float*>(w + 2 * feat + 2 * pos);
    p.fwt = reinterpret_cast<float*>(w + 2 * feat + 3 * pos);
    p.keep = reinterpret_cast<float*>(w + 2 * feat + 4 * pos);
    return p;
}

// One workgroup per window row: the 2 L feature softmaxes (one per thread),
// the decays and write weights with the keys', the cumulative log-decay
// (memory.py:108; wave 0: each lane sums its run of positions, an inclusive
// wave scan of the run sums places it), then the prior and final-write
// weights. Dynamic LDS: 3 L floats.
template <int MAXM, typename PT>
__global__ __launch_bounds__(256) void assoc_prep_kernel(
    const PT* __restrict__ proj, int64_t stride, int64_t fk_off, int64_t fq_off, int64_t decay_off,
    int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid, AssocPrep prep, int L,
    int M, const float* __restrict__ novelty, float refine_rate) {
    extern __shared__ float sh[];
    float* logd = sh;       // [L]
    float* cum = sh + L;    // [L]
    float* wt = sh + 2 * L;  // [L]
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const PT* rows0 = proj + b * L * stride;
    for (int job = tid; job < 2 * L; job += 256) {
        const bool query = job >= L;
        const int t = query ? job - L : job;
        const PT* row = rows0 + t * stride;
        const int64_t off = query ? fq_off : fk_off;
        float z[MAXM];
        float mx = -INFINITY;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) z[m] = to_f32(row[off + min(m, M - 1)]);  // unconditional, then masked
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
        float* dst = (query ? prep.qf : prep.kf) + (b * L + t) * MAXM;
#pragma unroll
        for (int m = 0; m < MAXM; m += 4)
            *reinterpret_cast<float4*>(dst + m) = make_float4(z[m] * inv, z[m + 1] * inv, z[m + 2] * inv, z[m + 3] * inv);
        if (!query) {
            const bool ok = valid[b * L + t] != 0;
            float decay = kMinDecay + kDecaySpan * sigmoid_f(to_f32(row[decay_off]));
            const float sv = fminf(fmaxf(surprise[b * L + t], 0.0f), 1.0f);
            float w = sigmoid_f(to_f32(row[write_off]));
            if (novelty != nullptr) {  // the refine terms (memory.py:257-268)
                decay = step::refine_decay(decay, refine_rate);
                w = w * sv * fminf(fmaxf(novelty[b * L + t], 0.0f), 1.0f);
            } else {
                w = w * (0.25f + 0.75f * sv);
            }
            logd[t] = ok ? logf(decay) : 0.0f;
            wt[t] = ok ? w : 0.0f;
        }
    }
    __syncthreads();
    if (wave == 0) {
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
    for (int s = tid; s < L; s += 256) {
        prep.cum[b * L + s] = cum[s];
        prep.prior[b * L + s] = cum[s] - logd[s];
        prep.wt[b * L + s] = wt[s];
        prep.fwt[b * L + s] = expf(total - cum[s]) * wt[s];
    }
    if (tid == 0) prep.keep[b] = expf(total);
}

// The window's own terms of the final state of a row, from the prepared
// weights: terms[d][m] = sum_s fwt_s tanh(v_s[d]) kf_s[m] on fp32 MFMA (A =
// the weighted values, 32 columns of a wave's half, B = the key features,
// K = slots, the slots split in two halves over wave pairs and added through
// LDS), normalizer terms sum_s fwt_s kf_s[m] by a wave reduction. FINAL
// writes the next state e^{c_{L-1}} state + terms (the fmaf the carry kernel
// applies between windows); otherwise the terms. Grid (rows, ceil(D / 64)).
template <int MAXM, bool FINAL, typename PT, bool TANH = true>
__global__ __launch_bounds__(256) void assoc_delta_kernel(
    const PT* __restrict__ proj, int64_t stride, int64_t value_off, AssocPrep prep,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ next_basis,
    float* __restrict__ next_normalizer, int L, int64_t D, int M) {
    extern __shared__ float sh[];
    constexpr int QP = MAXM + 1;
    float* fwt = sh;               // [L]
    float* kf = fwt + L;           // [L][QP]
    float* part = kf + L * QP;     // [2][16][64]
    const int64_t b = blockIdx.x;
    const int64_t c0 = static_cast<int64_t>(blockIdx.y) * 64;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int h = lane >> 5, r32 = lane & 31;
    for (int s = tid; s < L; s += 256) fwt[s] = prep.fwt[b * L + s];
    for (int i = tid; i < L * MAXM; i += 256) kf[(i / MAXM) * QP + i % MAXM] = prep.kf[b * L * MAXM + i];
    __syncthreads();
    const int half = ((L + 1) / 2 + 1) & ~1;
    const int db = wave & 1, kh = wave >> 1;
    const int s_lo = kh * half, s_hi = min(L, s_lo + half);
    const int64_t dv = c0 + db * 32 + r32;
    const PT* vcol = proj + b * L * stride + value_off + (dv < D ? dv : D - 1);
    const float fon = r32 < MAXM ? 1.0f : 0.0f;
    const int mf = min(r32, MAXM - 1);
    f32x16 acc = {};
    for (int s = s_lo; s < s_hi; s += 8) {  // four steps' operands loaded together
        float x[4], a[4], bf[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) x[q] = to_f32(vcol[min(s + 2 * q + h, L - 1) * stride]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int sl = s + 2 * q + h, slc = min(sl, L - 1);
            a[q] = sl < s_hi ? fwt[slc] * (TANH ? fast_tanh(x[q]) : x[q]) : 0.0f;
            bf[q] = kf[slc * QP + mf] * fon;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = mfma2(a[q], bf[q], acc);
    }
    if (kh == 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) part[(db * 16 + i) * kWave + lane] = acc[i];
    }
    __syncthreads();
    const float keep = prep.keep[b];
    if (kh == 0) {
        const int m = r32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t d = c0 + db * 32 + 8 * (i / 4) + 4 * h + (i % 4);
            if (m >= M || d >= D) continue;
            const int64_t at = (b * D + d) * M + m;
            const float terms = acc[i] + part[(db * 16 + i) * kWave + lane];
            next_basis[at] = FINAL ? fmaf(keep, basis[at], terms) : terms;
        }
    }
    if (blockIdx.y == 0 && wave == 3) {
        for (int m = 0; m < M; ++m) {
            float sum = 0.0f;
            for (int s = lane; s < L; s += kWave) sum = fmaf(fwt[s], kf[s * QP + m], sum);
            sum = wave_sum_xor(sum);
            if (lane == 0) next_normalizer[b * M + m] = FINAL ? fmaf(keep, normalizer[b * M + m], sum) : sum;
        }
    }
}

// The reads of a window row from its carried state: one workgroup per (row,
// group of kReadTiles 64-column tiles, 64 queries). It stages the prepared
// features and weights of its queries and of the slots that can reach them,
// forms the influence of slot s on query t,
//   e^{prior_t - c_s} (q_t . f_s) weight_s  (s < t, else 0),
// on fp32 MFMA (32 x 32 blocks, K = features) into LDS, and the denominators
// den_t = sum_s influence + e^{prior_t} (q_t . normalizer) by wave
// reductions. Then per column tile each wave forms a 32 x 32 block of
// sum_s influence tanh(v_s[d]) + e^{prior_t} (q_t . basis_d) on MFMA (A from
// LDS, B the value columns straight from memory, eight steps' loads in flight
// ahead of their use), and writes read = den/(den + 2^-8) num/(den + 2^-8).
constexpr int kReadTiles = 4;
constexpr int kReadRows = 64;
inline size_t read_lds(int64_t L, int64_t M) {
    const int64_t Lq = (L + 31) & ~int64_t(31), X = assoc_maxm(M);
    return static_cast<size_t>(kReadRows * (Lq + 1) + X * (Lq + 1) + kReadRows * (X + 1) + 2 * Lq + 2 * kReadRows) *
           sizeof(float);
}

template <int MAXM, typename PT, typename OutT, bool VEC4, bool TANH = true>
__global__ __launch_bounds__(256) void assoc_window_read_kernel(
    const PT* __restrict__ proj, int64_t stride, int64_t value_off, AssocPrep prep,
    const float* __restrict__ basis, const float* __restrict__ normalizer, OutT* __restrict__ out, int64_t ostride,
    int L, int64_t D, int M) {
    extern __shared__ float sh[];
    constexpr int QP = MAXM + 1;
    const int Lq = (L + 31) & ~31;
    const int IP = Lq + 1;
    float* infl = sh;                     // [64][IP]
    float* f_sh = infl + kReadRows * IP;  // [MAXM][IP]
    float* q_sh = f_sh + MAXM * IP;       // [64][QP]
    float* cum = q_sh + kReadRows * QP;   // [Lq]
    float* wt = cum + Lq;                 // [Lq]
    float* pr = wt + Lq;                  // [64] prior of the tile's queries
    float* den = pr + kReadRows;          // [64]
    const int64_t b = blockIdx.x;
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int h = lane >> 5, r32 = lane & 31;
    const int t0 = static_cast<int>(blockIdx.z) * kReadRows;
    const int rows = min(kReadRows, L - t0);
    const int s_cnt = t0 + rows;  // slots that can reach these queries (s < t <= t0 + rows - 1)
    // bf16 path: this lane's value columns, and the loads of its first eight
    // K steps, issued before the staging so that their latency passes under
    // it.
    const PT* vrows = proj + b * L * stride + value_off;
    const int64_t v_d0 = static_cast<int64_t>(blockIdx.y) * (kReadTiles * 64) + wave * 64;
    const int64_t v_dcol = v_d0 + 2 * r32;
    const int64_t v_dq = v_dcol < D ? v_dcol : 0;
    auto load2 = [&](const PT* p) {
        if constexpr (std::is_same<PT, float>::value) {
            return *reinterpret_cast<const float2*>(p);
        } else {
            const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
            return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
        }
    };
    float2 bn[8];
    if constexpr (VEC4) {
        if (v_d0 < D) {
#pragma unroll
            for (int u = 0; u < 8; ++u) bn[u] = load2(vrows + v_dq + min(2 * u + h, L - 1) * stride);
        }
    }
    for (int i = tid; i < s_cnt * MAXM; i += 256) f_sh[(i % MAXM) * IP + i / MAXM] = prep.kf[b * L * MAXM + i];
    for (int i = tid; i < kReadRows * MAXM; i += 256) {
        const int r = i / MAXM;
        q_sh[r * QP + i % MAXM] = r < rows ? prep.qf[(b * L + t0) * MAXM + i] : 0.0f;
    }
    for (int s2 = tid; s2 < s_cnt; s2 += 256) {
        cum[s2] = prep.cum[b * L + s2];
        wt[s2] = prep.wt[b * L + s2];
    }
    if (tid < kReadRows) pr[tid] = tid < rows ? prep.prior[b * L + t0 + tid] : 0.0f;
    __syncthreads();

    const int nsb = (s_cnt + 31) / 32;
    for (int blk = wave; blk < 2 * nsb; blk += 4) {
        const int tb = blk / nsb, sb = blk - tb * nsb;
        const int ra = tb * 32 + r32;
        const int s = sb * 32 + r32, sc = min(s, s_cnt - 1);
        f32x16 acc = {};
#pragma unroll
        for (int kk = 0; kk < MAXM / 2; ++kk) acc = mfma2(q_sh[ra * QP + 2 * kk + h], f_sh[(2 * kk + h) * IP + sc], acc);
        const float cs = cum[sc], ws = wt[sc];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = tb * 32 + 8 * (i / 4) + 4 * h + (i % 4);
            const float v = fast_exp(pr[r] - cs) * acc[i] * ws;
            infl[r * IP + s] = (s < t0 + r && r < rows) ? v : 0.0f;
        }
    }
    __syncthreads();
    for (int rr = 0; rr < kReadRows / 4; ++rr) {
        const int r = wave * (kReadRows / 4) + rr;
        float sum = 0.0f;
        for (int s = lane; s < s_cnt; s += kWave) sum += infl[r * IP + s];
        float nq = lane < M ? q_sh[r * QP + lane] * normalizer[b * M + lane] : 0.0f;
        sum = wave_sum_xor(sum);
        nq = wave_sum_xor(nq);
        if (lane == 0) den[r] = sum + fast_exp(pr[r]) * nq;
    }
    __syncthreads();

    const int kfull = (s_cnt + 1) & ~1;
    if constexpr (VEC4) {
        // Wave w: all 64 queries (m-tiles tb = 0, 1) x 64 columns d0 + 2 r + c
        // (n-tile c = 0, 1) as four 32x32 MFMA tiles, so each value's tanh is
        // formed once per workgroup; lane (r, h) feeds columns 2 r, 2 r + 1 of
        // one 2-column load of a value row (eight steps' loads in flight ahead
        // of their use). Slot s reaches query t only for s < t, so m-tile 0
        // (queries t0 .. t0 + 31) stops at slot t0 + 32 (exactly the sums of
        // the full range).
        if (v_d0 >= D) return;
        const int64_t dcol = v_dcol;
        const bool cok = dcol < D;  // D is a multiple of 4, so dcol + 1 < D too
        const PT* vcol = vrows + v_dq;
        const int k_end0 = min(kfull, t0 + 32);
        const float* ia0 = infl + r32 * IP + h;
        const float* ia1 = infl + (32 + r32) * IP + h;
        f32x16 acc[2][2];
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int c = 0; c < 2; ++c) acc[m][c] = f32x16{};
        for (int s = 0; s < kfull; s += 16) {
            float2 bc[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) bc[u] = bn[u];
            if (s + 16 < kfull) {
#pragma unroll
                for (int u = 0; u < 8; ++u) bn[u] = load2(vcol + min(s + 16 + 2 * u + h, L - 1) * stride);
            }
            const bool first = s < k_end0;  // wave-uniform
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float tx = TANH ? fast_tanh(bc[u].x) : bc[u].x, ty = TANH ? fast_tanh(bc[u].y) : bc[u].y;
                if (first) {
                    const float a0 = s + 2 * u + h < k_end0 ? ia0[s + 2 * u] : 0.0f;
                    acc[0][0] = mfma2(a0, tx, acc[0][0]);
                    acc[0][1] = mfma2(a0, ty, acc[0][1]);
                }
                const float a1 = s + 2 * u + h < kfull ? ia1[s + 2 * u] : 0.0f;
                acc[1][0] = mfma2(a1, tx, acc[1][0]);
                acc[1][1] = mfma2(a1, ty, acc[1][1]);
            }
        }
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const float ep = fast_exp(pr[m * 32 + r32]);
#pragma unroll
            for (int kk = 0; kk < MAXM / 2; ++kk) {
                const int mm = 2 * kk + h;
                const float on = mm < M ? 1.0f : 0.0f;
                const float aq = ep * q_sh[(m * 32 + r32) * QP + mm];
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    acc[m][c] = mfma2(aq, basis[(b * D + min(v_dq + c, D - 1)) * M + min(mm, M - 1)] * on, acc[m][c]);
            }
        }
        if (cok) {
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int rr = m * 32 + 8 * (i / 4) + 4 * h + (i % 4);
                    if (rr >= rows) continue;
                    // read = den / reg * num / reg, reg = den + 2^-8: the
                    // row's scale once (two divisions, no overflow of reg^2)
                    // for every column.
                    const float dn = den[rr], reg = dn + kReadEpsilon;
                    const float sc = (dn / reg) / reg;
                    OutT* o = out + (b * L + t0 + rr) * ostride + dcol;
                    o[0] = from_f32<OutT>(acc[m][0][i] * sc);
                    o[1] = from_f32<OutT>(acc[m][1][i] * sc);
                }
        }
        return;
    }
    const int tb = wave >> 1;
    // The wave's queries are t0 + tb * 32 .. + 31, and slot s reaches query t
    // only for s < t: past slot t0 + tb * 32 + 31 every influence is zero, so
    // the wave's products stop there (exactly the sums of the full range).
    const int k_end = min(kfull, t0 + tb * 32 + 32);
    const float* ia = infl + (tb * 32 + r32) * IP + h;
    const float ep = fast_exp(pr[tb * 32 + r32]);
    const int db = wave & 1;
    for (int ct = 0; ct < kReadTiles; ++ct) {
        const int64_t d0 = (static_cast<int64_t>(blockIdx.y) * kReadTiles + ct) * 64 + db * 32;
        if (d0 >= D) break;
        const int64_t dq = min(d0 + r32, D - 1);
        const PT* vcol = vrows + dq;
        f32x16 acc = {};
        float bn[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) bn[u] = to_f32(vcol[min(2 * u + h, L - 1) * stride]);
        for (int s = 0; s < k_end; s += 16) {
            float bc[8], av[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) bc[u] = bn[u];
            if (s + 16 < k_end) {
#pragma unroll
                for (int u = 0; u < 8; ++u) bn[u] = to_f32(vcol[min(s + 16 + 2 * u + h, L - 1) * stride]);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) av[u] = s + 2 * u + h < k_end ? ia[s + 2 * u] : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = mfma2(av[u], TANH ? fast_tanh(bc[u]) : bc[u], acc);
        }
#pragma unroll
        for (int kk = 0; kk < MAXM / 2; ++kk) {
            const int m = 2 * kk + h;
            const float on = m < M ? 1.0f : 0.0f;
            acc = mfma2(ep * q_sh[(tb * 32 + r32) * QP + m], basis[(b * D + dq) * M + min(m, M - 1)] * on, acc);
        }
        const int64_t d = d0 + r32;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = tb * 32 + 8 * (i / 4) + 4 * h + (i % 4);
            if (r >= rows || d >= D) continue;
            const float dn = den[r], reg = dn + kReadEpsilon;
            out[(b * L + t0 + r) * ostride + d] = from_f32<OutT>(acc[i] * ((dn / reg) / reg));
        }
    }
}

// The state carried into each of a sequence's windows and the state after the
// last: for element e of the flattened basis (D x M, then the M normalizer
// entries) of batch row b, cur = state_0; window w receives cur, then
// cur = fmaf(keep_w, cur, delta_w), the update the one-window entry applies at
// the end of a window (so the carried states equal a window-by-window run's).
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

// The three launches of a window's (or every window's) memory: prepare, the
// state terms (FINAL: the next state), the reads. Rows are batch rows (one
// window) or (batch row, window) pairs.
template <int MAXM, typename PT>
int launch_prep(const PT* proj, int64_t stride, int64_t fk_off, int64_t fq_off, int64_t decay_off,
                int64_t write_off, const float* surprise, const uint8_t* valid, const AssocPrep& prep, int64_t rows,
                int L, int M, hipStream_t s, const float* novelty = nullptr, float refine_rate = 0.0f) {
    hipLaunchKernelGGL((assoc_prep_kernel<MAXM, PT>), dim3(static_cast<unsigned>(rows)), dim3(256),
                       3 * static_cast<size_t>(L) * sizeof(float), s, proj, stride, fk_off, fq_off, decay_off,
                       write_off, surprise, valid, prep, L, M, novelty, refine_rate);
    return check_launch("associative memory (prepare)");
}

template <int MAXM, bool FINAL, typename PT, bool TANH = true>
int launch_delta(const PT* proj, int64_t stride, int64_t value_off, const AssocPrep& prep, const float* basis,
                 const float* normalizer, float* nb, float* nn, int64_t rows, int L, int64_t D, int M,
                 hipStream_t s) {
    const size_t lds = (static_cast<size_t>(L) * (MAXM + 2) + 2 * 16 * kWave) * sizeof(float);
    hipLaunchKernelGGL((assoc_delta_kernel<MAXM, FINAL, PT, TANH>), dim3(static_cast<unsigned>(rows),
                       static_cast<unsigned>((D + 63) / 64)), dim3(256), lds, s, proj, stride, value_off, prep, basis,
                       normalizer, nb, nn, L, D, M);
    return check_launch("associative memory (state terms)");
}

template <int MAXM, typename PT, bool TANH = true>
int launch_window_read(const PT* proj, int64_t stride, int64_t value_off, const AssocPrep& prep,
                       const float* basis, const float* normalizer, void* out, int out_dtype, int64_t ostride,
                       int64_t rows, int L, int64_t D, int M, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>((D + 64 * kReadTiles - 1) / (64 * kReadTiles)),
                    static_cast<unsigned>((L + kReadRows - 1) / kReadRows));
    // four columns per lane where every value row and output row starts at a
    // multiple of four elements (aligned 4-element loads and stores)
    const bool vec4 = D % 4 == 0 && stride % 4 == 0 && value_off % 4 == 0 && ostride % 4 == 0 &&
                      reinterpret_cast<uintptr_t>(proj) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
    auto launch = [&](auto kernel, auto* o) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), read_lds(L, M), s, proj, stride, value_off, prep, basis,
                           normalizer, o, ostride, L, D, M);
    };
    if (out_dtype == KOEMI_BF16) {
        if (vec4) launch(assoc_window_read_kernel<MAXM, PT, bf16, true, TANH>, static_cast<bf16*>(out));
        else launch(assoc_window_read_kernel<MAXM, PT, bf16, false, TANH>, static_cast<bf16*>(out));
    } else {
        if (vec4) launch(assoc_window_read_kernel<MAXM, PT, float, true, TANH>, static_cast<float*>(out));
        else launch(assoc_window_read_kernel<MAXM, PT, float, false, TANH>, static_cast<float*>(out));
    }
    return check_launch("associative memory (reads)");
}

inline size_t delta_lds(int64_t L, int64_t M) {
    return (static_cast<size_t>(L) * (assoc_maxm(M) + 2) + 2 * 16 * kWave) * sizeof(float);
}

// One-position window (a decode step): assoc_step_body (the shared header).
template <int MAXM, typename PT>
__global__ __launch_bounds__(256) void assoc_step_kernel(
    const PT* __restrict__ proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
    int64_t decay_off, int64_t write_off, const float* __restrict__ surprise, const uint8_t* __restrict__ valid,
    const float* __restrict__ basis, const float* __restrict__ normalizer, float* __restrict__ out,
    float* __restrict__ next_basis, float* __restrict__ next_normalizer, int64_t D, int M,
    const float* __restrict__ novelty = nullptr, float refine_rate = 0.0f, const float* __restrict__ fast = nullptr) {
    step::assoc_step_body<MAXM, PT>(proj, stride, value_off, fk_off, fq_off, decay_off, write_off, surprise, valid,
                                    basis, normalizer, out, next_basis, next_normalizer, D, M, blockIdx.x,
                                    static_cast<int>(blockIdx.y), novelty, refine_rate, fast);
}

// The refine memory's values (memory.py:266-267 with network.py:358): the
// value tanh(v) of each position (the same fast_tanh as the fast reads)
// minus the position's fast read, clamped to [-2, 2], as a dense fp32 [rows,
// D] array the state-terms and read kernels take in place of the projection's
// value columns (their TANH = false instances).
template <typename PT, typename FT>
__global__ __launch_bounds__(256) void refine_error_kernel(const PT* __restrict__ proj, int64_t stride,
                                                           int64_t value_off, const FT* __restrict__ fast,
                                                           int64_t fstride, float* __restrict__ err, int64_t rows,
                                                           int64_t D) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= rows * D) return;
    const int64_t r = i / D, d = i - r * D;
    err[i] = step::refine_value(fast_tanh(to_f32(proj[r * stride + value_off + d])), to_f32(fast[r * fstride + d]));
}

}  // namespace
}  // namespace koemi

using namespace koemi;

namespace {

// Largest window the LDS of the read kernel holds (64 influence rows of
// L + 1 floats plus the staged features and weights).
inline bool window_fits(int64_t L, int64_t M) { return read_lds(L, M) <= 160 * 1024 && delta_lds(L, M) <= 160 * 1024; }

struct WindowsWorkspace {
    size_t delta_basis, delta_norm, carried_basis, carried_norm, prep, total;
};

inline WindowsWorkspace windows_workspace(int64_t rows, int64_t window, int64_t width, int64_t features) {
    WindowsWorkspace w;
    const size_t basis_bytes = align256(static_cast<size_t>(rows * width * features) * sizeof(float));
    const size_t norm_bytes = align256(static_cast<size_t>(rows * features) * sizeof(float));
    w.delta_basis = 0;
    w.delta_norm = w.delta_basis + basis_bytes;
    w.carried_basis = w.delta_norm + norm_bytes;
    w.carried_norm = w.carried_basis + basis_bytes;
    w.prep = w.carried_norm + norm_bytes;
    w.total = w.prep + prep_bytes(rows, window, features);
    return w;
}

int check_assoc_args(int64_t row_stride, int64_t value_offset, int64_t feature_offset, int64_t query_feature_offset,
                     int64_t decay_offset, int64_t write_offset, int64_t width, int64_t features) {
    if (features > 32) return fail(KOEMI_ERR_UNSUPPORTED, "associative read supports at most 32 memory features");
    auto inside = [&](int64_t off, int64_t span) { return off >= 0 && off + span <= row_stride; };
    if (!inside(value_offset, width) || !inside(feature_offset, features) ||
        !inside(query_feature_offset, features) || !inside(decay_offset, 1) || !inside(write_offset, 1))
        return fail(KOEMI_ERR_INVALID, "associative read column offsets must lie inside the row stride");
    return KOEMI_OK;
}

// prepare, state terms (FINAL: next state from the given one), reads from the
// given (carried) state
template <int MAXM, bool FINAL, typename PT>
int run_window_memory(const PT* proj, int64_t stride, int64_t value_off, int64_t fk_off, int64_t fq_off,
                      int64_t decay_off, int64_t write_off, const float* surprise, const uint8_t* valid,
                      const AssocPrep& prep, const float* state_basis, const float* state_norm, float* nb, float* nn,
                      const float* read_basis, const float* read_norm, void* read, int read_dtype, int64_t ostride,
                      int64_t rows, int L, int64_t D, int M, hipStream_t s, bool reads) {
    int st = launch_prep<MAXM>(proj, stride, fk_off, fq_off, decay_off, write_off, surprise, valid, prep, rows, L, M, s);
    if (st != KOEMI_OK) return st;
    st = launch_delta<MAXM, FINAL>(proj, stride, value_off, prep, state_basis, state_norm, nb, nn, rows, L, D, M, s);
    if (st != KOEMI_OK || !reads) return st;
    return launch_window_read<MAXM>(proj, stride, value_off, prep, read_basis, read_norm, read, read_dtype, ostride, rows,
                                    L, D, M, s);
}

// Calls f with the projections as the given dtype's pointer (fp32 or bf16).
template <typename F>
int with_projection(const void* projections, int dtype, F&& f) {
    if (dtype == KOEMI_BF16) return f(static_cast<const bf16*>(projections));
    return f(static_cast<const float*>(projections));
}

}  // namespace

extern "C" size_t koemi_assoc_scan_read_workspace_bytes(int64_t batch, int64_t length, int64_t width,
                                                         int64_t features) {
    if (batch <= 0 || length <= 1 || width < 1 || features < 1) return 0;
    return prep_bytes(batch, length, features);
}

extern "C" int koemi_assoc_scan_read(const void* projections, int projection_dtype, int64_t row_stride, int64_t value_offset,
                                     int64_t feature_offset, int64_t query_feature_offset, int64_t decay_offset,
                                     int64_t write_offset, const float* surprise, const uint8_t* valid,
                                     const float* basis, const float* normalizer, void* read, int read_dtype,
                                     int64_t read_row_stride, float* next_basis, float* next_normalizer, int64_t batch,
                                     int64_t length, int64_t width, int64_t features, void* workspace,
                                     size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "associative read needs non-negative batch and length, positive width and features");
    int st = check_assoc_args(row_stride, value_offset, feature_offset, query_feature_offset, decay_offset,
                              write_offset, width, features);
    if (st != KOEMI_OK) return st;
    if (projection_dtype != KOEMI_F32 && projection_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read projections must be float32 or bfloat16");
    if (read_dtype != KOEMI_F32 && read_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative reads must be float32 or bfloat16");
    if (read_row_stride == 0) read_row_stride = width;
    if (read_row_stride < width) return fail(KOEMI_ERR_INVALID, "associative read row stride below the width");
    if (length == 1 && (read_dtype != KOEMI_F32 || read_row_stride != width))
        return fail(KOEMI_ERR_UNSUPPORTED, "a one-position associative read writes contiguous float32 reads");
    if (batch == 0 || length == 0) return KOEMI_OK;
    if (!window_fits(length, features))
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read window too long (%lld positions)",
                    static_cast<long long>(length));
    if (batch > 0x7fffffffLL || (width + 63) / 64 > 65535)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read grid too large");
    if (!projections || !surprise || !valid || !basis || !normalizer || !read || !next_basis || !next_normalizer)
        return fail(KOEMI_ERR_INVALID, "associative read received a null pointer");
    const hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(features);
    if (length == 1) {
        const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((width + 255) / 256));
        return with_projection(projections, projection_dtype, [&](auto proj) {
            using PT = std::remove_const_t<std::remove_pointer_t<decltype(proj)>>;
            auto step = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, proj, row_stride, value_offset, feature_offset,
                                   query_feature_offset, decay_offset, write_offset, surprise, valid, basis, normalizer,
                                   static_cast<float*>(read), next_basis, next_normalizer, width, M,
                                   static_cast<const float*>(nullptr), 0.0f, static_cast<const float*>(nullptr));
            };
            if (M <= 16) step(assoc_step_kernel<16, PT>);
            else step(assoc_step_kernel<32, PT>);
            return check_launch("koemi_assoc_scan_read");
        });
    }
    const size_t need = prep_bytes(batch, length, features);
    if (!workspace || workspace_bytes < need)
        return fail(KOEMI_ERR_INVALID, "associative read workspace too small: need %zu bytes", need);
    const AssocPrep prep = prep_at(workspace, batch, length, features);
    const int L = static_cast<int>(length);
    return with_projection(projections, projection_dtype, [&](auto proj) {
        if (M <= 16)
            return run_window_memory<16, true>(proj, row_stride, value_offset, feature_offset, query_feature_offset,
                                               decay_offset, write_offset, surprise, valid, prep, basis, normalizer,
                                               next_basis, next_normalizer, basis, normalizer, read, read_dtype,
                                               read_row_stride, batch, L, width, M, s, true);
        return run_window_memory<32, true>(proj, row_stride, value_offset, feature_offset, query_feature_offset,
                                           decay_offset, write_offset, surprise, valid, prep, basis, normalizer,
                                           next_basis, next_normalizer, basis, normalizer, read, read_dtype,
                                           read_row_stride, batch, L, width, M, s, true);
    });
}

extern "C" size_t koemi_assoc_scan_read_windows_workspace_bytes(int64_t batch, int64_t windows, int64_t window,
                                                                 int64_t width, int64_t features) {
    if (batch < 0 || windows < 0 || window < 1 || width < 1 || features < 1) return 0;
    return windows_workspace(batch * windows, window, width, features).total;
}

extern "C" int koemi_assoc_scan_read_windows(const void* projections, int projection_dtype, int64_t row_stride,
                                             int64_t value_offset,
                                             int64_t feature_offset, int64_t query_feature_offset,
                                             int64_t decay_offset, int64_t write_offset, const float* surprise,
                                             const uint8_t* valid, const float* basis, const float* normalizer,
                                             void* read, int read_dtype, int64_t read_row_stride, float* next_basis,
                                             float* next_normalizer, int64_t batch, int64_t windows, int64_t window,
                                             int64_t width, int64_t features, void* workspace, size_t workspace_bytes,
                                             koemi_stream_t stream) {
    if (batch < 0 || windows < 0 || window < 2 || width < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "windowed associative read needs non-negative batch and windows, a window of at "
                    "least two positions, positive width and features");
    int st = check_assoc_args(row_stride, value_offset, feature_offset, query_feature_offset, decay_offset,
                              write_offset, width, features);
    if (st != KOEMI_OK) return st;
    if (projection_dtype != KOEMI_F32 && projection_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read projections must be float32 or bfloat16");
    if (read_dtype != KOEMI_F32 && read_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative reads must be float32 or bfloat16");
    if (read_row_stride == 0) read_row_stride = width;
    if (read_row_stride < width) return fail(KOEMI_ERR_INVALID, "associative read row stride below the width");
    const int64_t rows = batch * windows;
    if (batch == 0) return KOEMI_OK;
    if (!window_fits(window, features))
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read window too long (%lld positions)",
                    static_cast<long long>(window));
    if (rows > 0x7fffffffLL || (width + 63) / 64 > 65535 || (width * features + features + 255) / 256 > 65535)
        return fail(KOEMI_ERR_UNSUPPORTED, "windowed associative read grid too large");
    if (!basis || !normalizer || !next_basis || !next_normalizer ||
        (windows > 0 && (!projections || !surprise || !valid || !read)))
        return fail(KOEMI_ERR_INVALID, "windowed associative read received a null pointer");
    const WindowsWorkspace ws = windows_workspace(rows, window, width, features);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "windowed associative read workspace too small: need %zu bytes", ws.total);
    char* w = static_cast<char*>(workspace);
    float* delta_basis = reinterpret_cast<float*>(w + ws.delta_basis);
    float* delta_norm = reinterpret_cast<float*>(w + ws.delta_norm);
    float* carried_basis = reinterpret_cast<float*>(w + ws.carried_basis);
    float* carried_norm = reinterpret_cast<float*>(w + ws.carried_norm);
    const AssocPrep prep = prep_at(w + ws.prep, rows, window, features);
    const hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(features);
    const int L = static_cast<int>(window);
    if (windows > 0) {
        // 1. every window's prepared weights and own terms of the final state (from a zero state)
        st = with_projection(projections, projection_dtype, [&](auto proj) {
            if (M <= 16)
                return run_window_memory<16, false>(proj, row_stride, value_offset, feature_offset,
                                                    query_feature_offset, decay_offset, write_offset, surprise, valid,
                                                    prep, nullptr, nullptr, delta_basis, delta_norm, nullptr, nullptr,
                                                    nullptr, KOEMI_F32, width, rows, L, width, M, s, false);
            return run_window_memory<32, false>(proj, row_stride, value_offset, feature_offset, query_feature_offset,
                                                decay_offset, write_offset, surprise, valid, prep, nullptr, nullptr,
                                                delta_basis, delta_norm, nullptr, nullptr, nullptr, KOEMI_F32, width,
                                                rows, L, width, M, s, false);
        });
        if (st != KOEMI_OK) return st;
    }
    // 2. the state carried into each window, and the final state
    const int64_t DM = width * features;
    hipLaunchKernelGGL(assoc_carry_kernel, dim3(static_cast<unsigned>(batch), static_cast<unsigned>((DM + M + 255) / 256)),
                       dim3(256), 0, s, delta_basis, delta_norm, prep.keep, basis, normalizer, carried_basis,
                       carried_norm, next_basis, next_normalizer, windows, DM, static_cast<int64_t>(M));
    st = check_launch("koemi_assoc_scan_read_windows(carry)");
    if (st != KOEMI_OK || windows == 0) return st;
    // 3. the reads of every window from its carried state
    return with_projection(projections, projection_dtype, [&](auto proj) {
        if (M <= 16)
            return launch_window_read<16>(proj, row_stride, value_offset, prep, carried_basis, carried_norm, read,
                                          read_dtype, read_row_stride, rows, L, width, M, s);
        return launch_window_read<32>(proj, row_stride, value_offset, prep, carried_basis, carried_norm, read,
                                      read_dtype, read_row_stride, rows, L, width, M, s);
    });
}

// ----------------------------------------------------------- refine memory ---
// The refine memory of the herm ablation (network.py:359-384): the same
// projection, features and query features as the fast memory, the refine
// write terms (memory.py:257-268: decay 1 - (1 - decay) rate capped at
// 1 - 2^-16, weight sigmoid(w) clamp(surprise) clamp(novelty), value
// clamp(tanh(v) - fast read, -2, 2), masked like the fast terms), read from
// and written into the refine basis and normalizer.
namespace {

// The refine values of `rows` x `length` positions into `err` (fp32, dense).
int launch_refine_error(const void* projections, int projection_dtype, int64_t row_stride, int64_t value_offset,
                        const void* fast, int fast_dtype, int64_t fast_row_stride, float* err, int64_t positions,
                        int64_t width, hipStream_t s) {
    const int64_t n = positions * width;
    if (n == 0) return KOEMI_OK;
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    return with_projection(projections, projection_dtype, [&](auto proj) {
        using PT = std::remove_const_t<std::remove_pointer_t<decltype(proj)>>;
        if (fast_dtype == KOEMI_BF16)
            hipLaunchKernelGGL((refine_error_kernel<PT, bf16>), grid, dim3(256), 0, s, proj, row_stride, value_offset,
                               static_cast<const bf16*>(fast), fast_row_stride, err, positions, width);
        else
            hipLaunchKernelGGL((refine_error_kernel<PT, float>), grid, dim3(256), 0, s, proj, row_stride, value_offset,
                               static_cast<const float*>(fast), fast_row_stride, err, positions, width);
        return check_launch("refine memory (values)");
    });
}

// prepare (refine terms), state terms from the refine values (FINAL: next
// state from the given one), reads from the given (carried) state.
template <int MAXM, bool FINAL, typename PT>
int run_refine_window_memory(const PT* proj, int64_t stride, int64_t fk_off, int64_t fq_off, int64_t decay_off,
                             int64_t write_off, const float* surprise, const uint8_t* valid, const float* novelty,
                             float rate, const float* err, const AssocPrep& prep, const float* state_basis,
                             const float* state_norm, float* nb, float* nn, const float* read_basis,
                             const float* read_norm, void* read, int read_dtype, int64_t ostride, int64_t rows, int L,
                             int64_t D, int M, hipStream_t s, bool reads) {
    int st = launch_prep<MAXM>(proj, stride, fk_off, fq_off, decay_off, write_off, surprise, valid, prep, rows, L, M, s,
                               novelty, rate);
    if (st != KOEMI_OK) return st;
    st = launch_delta<MAXM, FINAL, float, false>(err, D, 0, prep, state_basis, state_norm, nb, nn, rows, L, D, M, s);
    if (st != KOEMI_OK || !reads) return st;
    return launch_window_read<MAXM, float, false>(err, D, 0, prep, read_basis, read_norm, read, read_dtype, ostride,
                                                  rows, L, D, M, s);
}

int check_refine_args(const float* novelty, float rate, const void* fast, int fast_dtype, int64_t fast_row_stride,
                      int64_t width) {
    if (!(rate > 0.0f && rate <= 1.0f)) return fail(KOEMI_ERR_INVALID, "refine decay rate must be in (0, 1]");
    if (fast_dtype != KOEMI_F32 && fast_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "the fast reads must be float32 or bfloat16");
    if (fast_row_stride < width) return fail(KOEMI_ERR_INVALID, "fast read row stride below the width");
    if (!novelty || !fast) return fail(KOEMI_ERR_INVALID, "refine memory received a null pointer");
    return KOEMI_OK;
}

}  // namespace

extern "C" size_t koemi_assoc_refine_scan_read_workspace_bytes(int64_t batch, int64_t length, int64_t width,
                                                                int64_t features) {
    if (batch <= 0 || length <= 1 || width < 1 || features < 1) return 0;
    return prep_bytes(batch, length, features) + align256(static_cast<size_t>(batch * length * width) * sizeof(float));
}

extern "C" int koemi_assoc_refine_scan_read(
    const void* projections, int projection_dtype, int64_t row_stride, int64_t value_offset, int64_t feature_offset,
    int64_t query_feature_offset, int64_t decay_offset, int64_t write_offset, const float* surprise,
    const uint8_t* valid, const float* novelty, float refine_decay_rate, const void* fast_read, int fast_dtype,
    int64_t fast_row_stride, const float* basis, const float* normalizer, void* read, int read_dtype,
    int64_t read_row_stride, float* next_basis, float* next_normalizer, int64_t batch, int64_t length, int64_t width,
    int64_t features, void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "refine read needs non-negative batch and length, positive width and features");
    int st = check_assoc_args(row_stride, value_offset, feature_offset, query_feature_offset, decay_offset,
                              write_offset, width, features);
    if (st != KOEMI_OK) return st;
    if (fast_row_stride == 0) fast_row_stride = width;
    if (batch > 0 && length > 0 &&
        (st = check_refine_args(novelty, refine_decay_rate, fast_read, fast_dtype, fast_row_stride, width)) != KOEMI_OK)
        return st;
    if (projection_dtype != KOEMI_F32 && projection_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read projections must be float32 or bfloat16");
    if (read_dtype != KOEMI_F32 && read_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative reads must be float32 or bfloat16");
    if (read_row_stride == 0) read_row_stride = width;
    if (read_row_stride < width) return fail(KOEMI_ERR_INVALID, "associative read row stride below the width");
    if (length == 1 && (read_dtype != KOEMI_F32 || read_row_stride != width || fast_dtype != KOEMI_F32 ||
                        fast_row_stride != width))
        return fail(KOEMI_ERR_UNSUPPORTED, "a one-position refine read takes and writes contiguous float32 reads");
    if (batch == 0 || length == 0) return KOEMI_OK;
    if (!window_fits(length, features))
        return fail(KOEMI_ERR_UNSUPPORTED, "refine read window too long (%lld positions)", static_cast<long long>(length));
    if (batch > 0x7fffffffLL || (width + 63) / 64 > 65535 || batch * length * width > 0x7fffffffLL * 256)
        return fail(KOEMI_ERR_UNSUPPORTED, "refine read grid too large");
    if (!projections || !surprise || !valid || !basis || !normalizer || !read || !next_basis || !next_normalizer)
        return fail(KOEMI_ERR_INVALID, "refine read received a null pointer");
    const hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(features);
    if (length == 1) {
        const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((width + 255) / 256));
        return with_projection(projections, projection_dtype, [&](auto proj) {
            using PT = std::remove_const_t<std::remove_pointer_t<decltype(proj)>>;
            auto step = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, proj, row_stride, value_offset, feature_offset,
                                   query_feature_offset, decay_offset, write_offset, surprise, valid, basis, normalizer,
                                   static_cast<float*>(read), next_basis, next_normalizer, width, M, novelty,
                                   refine_decay_rate, static_cast<const float*>(fast_read));
            };
            if (M <= 16) step(assoc_step_kernel<16, PT>);
            else step(assoc_step_kernel<32, PT>);
            return check_launch("koemi_assoc_refine_scan_read");
        });
    }
    const size_t pb = prep_bytes(batch, length, features);
    const size_t need = koemi_assoc_refine_scan_read_workspace_bytes(batch, length, width, features);
    if (!workspace || workspace_bytes < need)
        return fail(KOEMI_ERR_INVALID, "refine read workspace too small: need %zu bytes", need);
    const AssocPrep prep = prep_at(workspace, batch, length, features);
    float* err = reinterpret_cast<float*>(static_cast<char*>(workspace) + pb);
    st = launch_refine_error(projections, projection_dtype, row_stride, value_offset, fast_read, fast_dtype,
                             fast_row_stride, err, batch * length, width, s);
    if (st != KOEMI_OK) return st;
    const int L = static_cast<int>(length);
    return with_projection(projections, projection_dtype, [&](auto proj) {
        if (M <= 16)
            return run_refine_window_memory<16, true>(proj, row_stride, feature_offset, query_feature_offset,
                                                      decay_offset, write_offset, surprise, valid, novelty,
                                                      refine_decay_rate, err, prep, basis, normalizer, next_basis,
                                                      next_normalizer, basis, normalizer, read, read_dtype,
                                                      read_row_stride, batch, L, width, M, s, true);
        return run_refine_window_memory<32, true>(proj, row_stride, feature_offset, query_feature_offset, decay_offset,
                                                  write_offset, surprise, valid, novelty, refine_decay_rate, err, prep,
                                                  basis, normalizer, next_basis, next_normalizer, basis, normalizer,
                                                  read, read_dtype, read_row_stride, batch, L, width, M, s, true);
    });
}

extern "C" size_t koemi_assoc_refine_scan_read_windows_workspace_bytes(int64_t batch, int64_t windows, int64_t window,
                                                                        int64_t width, int64_t features) {
    if (batch < 0 || windows < 0 || window < 1 || width < 1 || features < 1) return 0;
    return windows_workspace(batch * windows, window, width, features).total +
           align256(static_cast<size_t>(batch * windows * window * width) * sizeof(float));
}

extern "C" int koemi_assoc_refine_scan_read_windows(
    const void* projections, int projection_dtype, int64_t row_stride, int64_t value_offset, int64_t feature_offset,
    int64_t query_feature_offset, int64_t decay_offset, int64_t write_offset, const float* surprise,
    const uint8_t* valid, const float* novelty, float refine_decay_rate, const void* fast_read, int fast_dtype,
    int64_t fast_row_stride, const float* basis, const float* normalizer, void* read, int read_dtype,
    int64_t read_row_stride, float* next_basis, float* next_normalizer, int64_t batch, int64_t windows, int64_t window,
    int64_t width, int64_t features, void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || windows < 0 || window < 2 || width < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "windowed refine read needs non-negative batch and windows, a window of at "
                    "least two positions, positive width and features");
    int st = check_assoc_args(row_stride, value_offset, feature_offset, query_feature_offset, decay_offset,
                              write_offset, width, features);
    if (st != KOEMI_OK) return st;
    if (fast_row_stride == 0) fast_row_stride = width;
    if (batch > 0 && windows > 0 &&
        (st = check_refine_args(novelty, refine_decay_rate, fast_read, fast_dtype, fast_row_stride, width)) != KOEMI_OK)
        return st;
    if (projection_dtype != KOEMI_F32 && projection_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative read projections must be float32 or bfloat16");
    if (read_dtype != KOEMI_F32 && read_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "associative reads must be float32 or bfloat16");
    if (read_row_stride == 0) read_row_stride = width;
    if (read_row_stride < width) return fail(KOEMI_ERR_INVALID, "associative read row stride below the width");
    const int64_t rows = batch * windows;
    if (batch == 0) return KOEMI_OK;
    if (!window_fits(window, features))
        return fail(KOEMI_ERR_UNSUPPORTED, "refine read window too long (%lld positions)", static_cast<long long>(window));
    if (rows > 0x7fffffffLL || (width + 63) / 64 > 65535 || (width * features + features + 255) / 256 > 65535 ||
        rows * window * width > 0x7fffffffLL * 256)
        return fail(KOEMI_ERR_UNSUPPORTED, "windowed refine read grid too large");
    if (!basis || !normalizer || !next_basis || !next_normalizer ||
        (windows > 0 && (!projections || !surprise || !valid || !read)))
        return fail(KOEMI_ERR_INVALID, "windowed refine read received a null pointer");
    const WindowsWorkspace ws = windows_workspace(rows, window, width, features);
    const size_t need = koemi_assoc_refine_scan_read_windows_workspace_bytes(batch, windows, window, width, features);
    if (!workspace || workspace_bytes < need)
        return fail(KOEMI_ERR_INVALID, "windowed refine read workspace too small: need %zu bytes", need);
    char* w = static_cast<char*>(workspace);
    float* delta_basis = reinterpret_cast<float*>(w + ws.delta_basis);
    float* delta_norm = reinterpret_cast<float*>(w + ws.delta_norm);
    float* carried_basis = reinterpret_cast<float*>(w + ws.carried_basis);
    float* carried_norm = reinterpret_cast<float*>(w + ws.carried_norm);
    float* err = reinterpret_cast<float*>(w + ws.total);
    const AssocPrep prep = prep_at(w + ws.prep, rows, window, features);
    const hipStream_t s = as_stream(stream);
    const int M = static_cast<int>(features);
    const int L = static_cast<int>(window);
    if (windows > 0) {
        st = launch_refine_error(projections, projection_dtype, row_stride, value_offset, fast_read, fast_dtype,
                                 fast_row_stride, err, rows * window, width, s);
        if (st != KOEMI_OK) return st;
        st = with_projection(projections, projection_dtype, [&](auto proj) {
            if (M <= 16)
                return run_refine_window_memory<16, false>(proj, row_stride, feature_offset, query_feature_offset,
                                                           decay_offset, write_offset, surprise, valid, novelty,
                                                           refine_decay_rate, err, prep, nullptr, nullptr,
                                                           delta_basis, delta_norm, nullptr, nullptr, nullptr,
                                                           KOEMI_F32, width, rows, L, width, M, s, false);
            return run_refine_window_memory<32, false>(proj, row_stride, feature_offset, query_feature_offset,
                                                       decay_offset, write_offset, surprise, valid, novelty,
                                                       refine_decay_rate, err, prep, nullptr, nullptr, delta_basis,
                                                       delta_norm, nullptr, nullptr, nullptr, KOEMI_F32, width, rows,
                                                       L, width, M, s, false);
        });
        if (st != KOEMI_OK) return st;
    }
    const int64_t DM = width * features;
    hipLaunchKernelGGL(assoc_carry_kernel, dim3(static_cast<unsigned>(batch), static_cast<unsigned>((DM + M + 255) / 256)),
                       dim3(256), 0, s, delta_basis, delta_norm, prep.keep, basis, normalizer, carried_basis,
                       carried_norm, next_basis, next_normalizer, windows, DM, static_cast<int64_t>(M));
    st = check_launch("koemi_assoc_refine_scan_read_windows(carry)");
    if (st != KOEMI_OK || windows == 0) return st;
    if (M <= 16)
        return launch_window_read<16, float, false>(err, width, 0, prep, carried_basis, carried_norm, read, read_dtype,
                                                    read_row_stride, rows, L, width, M, s);
    return launch_window_read<32, float, false>(err, width, 0, prep, carried_basis, carried_norm, read, read_dtype,
                                                read_row_stride, rows, L, width, M, s);
}
