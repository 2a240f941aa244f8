/*
 * koemi_oracle.c — CPU restatement of the Koemi-5HOM HERM hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (koemi-5hom_amd/) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, as the checker and the CPU baseline.
 *
 * Build: oracle/build.py (gcc -O3 -ffp-contract=off). Contraction is off so
 * that every a*b+c here is two roundings unless fmaf() is written explicitly,
 * exactly as the statements read.
 *
 * Functions and the reference lines they restate:
 *   oracle_scan_sequential_{f32,f64}  tests/model/test_scan.py:10-16,
 *       tests/cuda/test_dense_cuda.py:21-33 (state = a_t * state + b_t, in the
 *       tensor dtype, h_{-1} = initial; broadcast retention is one coefficient
 *       per (batch, position), dense/affine_scan.cu:46-48)
 *   oracle_det_expf / oracle_det_logf  the reproducible exp/log defined for the
 *       scores (Cody-Waite + Taylor; log via atanh series), stated step by step
 *   oracle_surprise_rows  model/network.py:677-688 and
 *       think/surprise_kernel.cu:84-134: nll = log(sum exp(z - max)) + max - z_t,
 *       s = 1 - exp(-nll / lnV), invalid -> 0, with the kernel's accumulation
 *       order: V <= 256, 16 lanes per row (lane l: j = u*64 + l*4 + p in (u, p)
 *       order) and a 16-lane pairwise tree; longer rows, 64 lanes (lane l:
 *       j = k*256 + l*4 + p in (k, p) order) and a 64-lane pairwise tree
 *   oracle_quantile  torch.quantile(s, q), linear: rank = q * (n - 1) in
 *       float32, lerp between the two order statistics (torch's lerp form)
 *   oracle_route_learned  model/router.py:46-49 (softmax then topk, ties to the
 *       lower index), left-to-right softmax sum
 *   oracle_rmsnorm_silu_f32  core/rmsnorm_silu.cu:62-91 in fp32 with libm expf
 *       (the CPU baseline port of the fused forward)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ scan --- */

void oracle_scan_sequential_f32(const float* a, const float* b, const float* h0, float* h, int64_t B, int64_t L,
                                int64_t F, int broadcast) {
    float* state = (float*)malloc((size_t)(F > 0 ? F : 1) * sizeof(float));
    for (int64_t bi = 0; bi < B; ++bi) {
        memcpy(state, h0 + bi * F, (size_t)F * sizeof(float));
        for (int64_t t = 0; t < L; ++t) {
            const float* bt = b + (bi * L + t) * F;
            float* ht = h + (bi * L + t) * F;
            if (broadcast) {
                const float at = a[bi * L + t];
                for (int64_t f = 0; f < F; ++f) {
                    const float prod = at * state[f];
                    state[f] = prod + bt[f];
                    ht[f] = state[f];
                }
            } else {
                const float* at = a + (bi * L + t) * F;
                for (int64_t f = 0; f < F; ++f) {
                    const float prod = at[f] * state[f];
                    state[f] = prod + bt[f];
                    ht[f] = state[f];
                }
            }
        }
    }
    free(state);
}

void oracle_scan_sequential_f64(const double* a, const double* b, const double* h0, double* h, int64_t B, int64_t L,
                                int64_t F, int broadcast) {
    double* state = (double*)malloc((size_t)(F > 0 ? F : 1) * sizeof(double));
    for (int64_t bi = 0; bi < B; ++bi) {
        memcpy(state, h0 + bi * F, (size_t)F * sizeof(double));
        for (int64_t t = 0; t < L; ++t) {
            const double* bt = b + (bi * L + t) * F;
            double* ht = h + (bi * L + t) * F;
            for (int64_t f = 0; f < F; ++f) {
                const double at = broadcast ? a[bi * L + t] : a[(bi * L + t) * F + f];
                state[f] = at * state[f] + bt[f];
                ht[f] = state[f];
            }
        }
    }
    free(state);
}

/* --------------------------------------------------------- exp and log --- */

static const float kLog2e = 1.4426950216293335f;
static const float kLn2Hi = 0.693145751953125f;
static const float kLn2Lo = 1.428606765330187e-06f;
static const float kSqrt2 = 1.4142135381698608f;

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}
static uint32_t float_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* e^x: x = n ln2 + r (n = rint(x log2e), r by two fmaf with the split ln2),
 * e^r by the degree-6 polynomial c6 .. c0 below (minimax relative error with
 * each coefficient rounded to fp32 in turn; c1 = c0 = 1) by Horner with fmaf,
 * times 2^n by ldexpf (exact: the result is normal for -86 <= x <= 88). */
float oracle_det_expf(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return INFINITY;
    const float n = rintf(x * kLog2e);
    float r = fmaf(-n, kLn2Hi, x);
    r = fmaf(-n, kLn2Lo, r);
    float p = 0.0013814611593261361f;   /* 0x3ab51225 */
    p = fmaf(p, r, 0.008368710055947304f);  /* 0x3c091cea */
    p = fmaf(p, r, 0.04166838899254799f);   /* 0x3d2aac79 */
    p = fmaf(p, r, 0.1666652113199234f);    /* 0x3e2aaa49 */
    p = fmaf(p, r, 0.4999999403953552f);    /* 0x3efffffe */
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* log x: x = m 2^e, m in [sqrt(1/2), sqrt(2)); log m = 2 atanh((m-1)/(m+1)). */
float oracle_det_logf(float x) {
    if (x != x) return x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (isinf(x)) return x;
    int e_adj = 0;
    if (x < 1.1754943508222875e-38f) {
        x = x * 16777216.0f;
        e_adj = -24;
    }
    const uint32_t u = float_to_bits(x);
    int e = (int)((u >> 23) & 0xffu) - 127 + e_adj;
    float m = bits_to_float((u & 0x007fffffu) | 0x3f800000u);
    if (m > kSqrt2) {
        m = m * 0.5f;
        e += 1;
    }
    const float f = (m - 1.0f) / (m + 1.0f);
    const float s = f * f;
    float p = 1.111111119389534e-01f;
    p = fmaf(p, s, 1.428571492433548e-01f);
    p = fmaf(p, s, 2.0000000298023224e-01f);
    p = fmaf(p, s, 3.333333432674408e-01f);
    const float fs = f * s;
    const float atanh_f = fmaf(fs, p, f);
    const float log_m = atanh_f * 2.0f;
    const float ef = (float)e;
    return fmaf(ef, kLn2Hi, fmaf(ef, kLn2Lo, log_m));
}

/* --------------------------------------------------------------- surprise --- */

/* Sum of the 64 lane partials: pairwise tree, lane l with lane l + off for
 * off = 32, 16, ..., 1 (the kernel's xor butterfly gives the same sums). */
static float tree64(float* v) {
    for (int off = 32; off > 0; off >>= 1)
        for (int l = 0; l < off; ++l) v[l] = v[l] + v[l + off];
    return v[0];
}

void oracle_surprise_rows(const float* logits, const float* bias, const int64_t* targets, const uint8_t* valid,
                          float* out, int64_t rows, int64_t V, float log_vocab) {
    const int64_t nchunks = (V + 255) / 256;
    for (int64_t r = 0; r < rows; ++r) {
        if (!valid[r]) {
            out[r] = 0.0f;
            continue;
        }
        const float* z = logits + r * V;
        float m = -INFINITY;
        for (int64_t j = 0; j < V; ++j) {
            const float zj = bias ? z[j] + bias[j] : z[j];
            m = fmaxf(m, zj);
        }
        float lane[64];
        float sum;
        if (V <= 256) {
            /* 16 lanes per row: lane l holds j = u*64 + l*4 + p, summed in (u, p)
               order, then a 16-lane pairwise tree */
            for (int l = 0; l < 16; ++l) {
                float acc = 0.0f;
                for (int u = 0; u < 4; ++u)
                    for (int p = 0; p < 4; ++p) {
                        const int64_t j = (int64_t)u * 64 + (int64_t)l * 4 + p;
                        if (j < V) {
                            const float zj = bias ? z[j] + bias[j] : z[j];
                            acc = acc + oracle_det_expf(zj - m);
                        }
                    }
                lane[l] = acc;
            }
            for (int off = 8; off > 0; off >>= 1)
                for (int l = 0; l < off; ++l) lane[l] = lane[l] + lane[l + off];
            sum = lane[0];
        } else {
            for (int l = 0; l < 64; ++l) {
                float acc = 0.0f;
                for (int64_t k = 0; k < nchunks; ++k)
                    for (int p = 0; p < 4; ++p) {
                        const int64_t j = k * 256 + (int64_t)l * 4 + p;
                        if (j < V) {
                            const float zj = bias ? z[j] + bias[j] : z[j];
                            acc = acc + oracle_det_expf(zj - m);
                        }
                    }
                lane[l] = acc;
            }
            sum = tree64(lane);
        }
        const int64_t t = targets[r];
        if (t < 0 || t >= V) {
            out[r] = NAN;
            continue;
        }
        const float zt = bias ? z[t] + bias[t] : z[t];
        const float nll = (oracle_det_logf(sum) + m) - zt;
        out[r] = 1.0f - oracle_det_expf(-nll / log_vocab);
    }
}

/* -------------------------------------------------------------- quantile --- */

static int cmp_float(const void* pa, const void* pb) {
    const float a = *(const float*)pa, b = *(const float*)pb;
    return (a > b) - (a < b);
}

/* torch.quantile(s, q) with linear interpolation; NaN if any score is NaN. */
float oracle_quantile(const float* s, int64_t n, float q) {
    float* sorted = (float*)malloc((size_t)n * sizeof(float));
    int has_nan = 0;
    for (int64_t i = 0; i < n; ++i) {
        sorted[i] = s[i];
        if (s[i] != s[i]) has_nan = 1;
    }
    if (has_nan) {
        free(sorted);
        return NAN;
    }
    qsort(sorted, (size_t)n, sizeof(float), cmp_float);
    const float rank = q * (float)(n - 1);
    const int64_t lo = (int64_t)rank;
    const int64_t hi = (int64_t)ceilf(rank);
    const float w = rank - (float)lo;
    const float a = sorted[lo], b = sorted[hi];
    free(sorted);
    return w < 0.5f ? fmaf(w, b - a, a) : fmaf(w - 1.0f, b - a, b);
}

/* ------------------------------------------------------------ learned route --- */

void oracle_route_learned(const float* logits, const uint8_t* valid, int64_t* idx, float* w, int64_t T, int64_t E,
                          int64_t k) {
    for (int64_t t = 0; t < T; ++t) {
        if (!valid[t]) {
            for (int64_t s = 0; s < k; ++s) {
                idx[t * k + s] = -1;
                w[t * k + s] = 0.0f;
            }
            continue;
        }
        const float* l = logits + t * E;
        float m = -INFINITY;
        for (int64_t j = 0; j < E; ++j) m = fmaxf(m, l[j]);
        float sum = 0.0f;
        for (int64_t j = 0; j < E; ++j) sum = sum + oracle_det_expf(l[j] - m);
        float prev_p = INFINITY;
        int64_t prev_j = -1;
        for (int64_t s = 0; s < k; ++s) {
            int64_t best = -1;
            float best_p = 0.0f;
            for (int64_t j = 0; j < E; ++j) {
                const float p = oracle_det_expf(l[j] - m) / sum;
                const int after = (p < prev_p) || (p == prev_p && j > prev_j);
                if (after && (best < 0 || p > best_p)) {
                    best = j;
                    best_p = p;
                }
            }
            idx[t * k + s] = best;
            w[t * k + s] = best < 0 ? 0.0f : best_p;
            prev_p = best_p;
            prev_j = best;
        }
    }
}

/* ------------------------------------------------------------- rmsnorm-silu --- */

void oracle_rmsnorm_silu_f32(const float* x, const float* w, float* y, float* inv_out, int64_t rows, int64_t H,
                             float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * H;
        float ss = 0.0f;
        for (int64_t c = 0; c < H; ++c) ss = fmaf(xr[c], xr[c], ss);
        const float inv = 1.0f / sqrtf(ss / (float)H + eps);
        inv_out[r] = inv;
        for (int64_t c = 0; c < H; ++c) {
            const float v = xr[c] * inv * w[c];
            y[r * H + c] = v / (1.0f + expf(-v));
        }
    }
}

/* Element-wise forms for accuracy sweeps. */
void oracle_det_expf_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_det_expf(x[i]);
}
void oracle_det_logf_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_det_logf(x[i]);
}
