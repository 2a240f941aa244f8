// Affine scan h_t = a_t * h_{t-1} + b_t for gfx950.
//
// Reference semantics: src/koemi/cuda_kernels/dense/affine_scan.cu:17-106 (one
// thread walks one column through the whole sequence). Here the scan is
// two-level so that a column is worked on by NSEG waves at once:
//
//   * A workgroup owns 64 consecutive state columns of one batch row (lane =
//     column, so every global access of a wave is one contiguous 64-element
//     row segment) and walks the sequence in chunks of CH = NSEG * S steps.
//   * Inside a chunk, wave w scans its S consecutive steps serially in
//     registers, producing the segment transfer (P = prod a, B = local scan).
//   * The NSEG segment transfers are composed through LDS,
//     (a2, b2) o (a1, b1) = (a2 a1, a2 b1 + b2), starting from the carried
//     state of the previous chunk, which stays in a register for the whole
//     sequence (no inter-workgroup traffic, no second pass over a and b).
//   * The next chunk's a/b are loaded before the current chunk is combined, so
//     two chunks of loads are in flight per wave.
//
// HBM traffic is the algorithmic minimum: read a and b once, write h once.
#include "common.hpp"

#include <type_traits>

namespace koemi {
namespace {

#ifndef KOEMI_SCAN_STEPS
#define KOEMI_SCAN_STEPS 8
#endif
#ifndef KOEMI_SCAN_SEGMENTS
#define KOEMI_SCAN_SEGMENTS 8
#endif
#ifndef KOEMI_SCAN_BUFFERS
#define KOEMI_SCAN_BUFFERS 3
#endif
constexpr int kScanSteps = KOEMI_SCAN_STEPS;        // S: serial steps per wave per chunk
constexpr int kScanSegments = KOEMI_SCAN_SEGMENTS;  // NSEG: waves per workgroup

// Loads are unconditional (the position is clamped into the sequence) and the
// identity element is selected afterwards: loads under divergent branches would
// force the compiler to wait for every outstanding load, including the prefetch
// of the next chunk.
template <typename T, typename A, int S, bool BCAST>
__device__ __forceinline__ void scan_load(const T* __restrict__ a_col, const T* __restrict__ b_col,
                                          int64_t a_stride, int64_t F, int64_t L, int64_t t_first,
                                          bool col_ok, A (&ra)[S], A (&rb)[S]) {
    T va[S], vb[S];
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int64_t t = t_first + i;
        const int64_t tc = t < L ? t : L - 1;
        va[i] = a_col[tc * a_stride];
        vb[i] = b_col[tc * F];
    }
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const bool ok = col_ok && t_first + i < L;
        ra[i] = ok ? static_cast<A>(va[i]) : A(1);
        rb[i] = ok ? static_cast<A>(vb[i]) : A(0);
    }
}

template <typename T, int S, int NSEG, bool BCAST>
__global__ __launch_bounds__(kWave * NSEG) void scan_forward_kernel(
    const T* __restrict__ a, const T* __restrict__ b, const T* __restrict__ h0, T* __restrict__ h,
    int64_t L, int64_t F, int64_t col_tiles) {
    using A = typename AccOf<T>::type;
    constexpr int CH = S * NSEG;
    __shared__ A seg_p[NSEG][kWave];
    __shared__ A seg_b[NSEG][kWave];

    const int lane = lane_id();
    const int seg = static_cast<int>(threadIdx.x) / kWave;
    const int64_t bi = static_cast<int64_t>(blockIdx.x) / col_tiles;
    const int64_t f = (static_cast<int64_t>(blockIdx.x) % col_tiles) * kWave + lane;
    const bool col_ok = f < F;
    const int64_t fc = col_ok ? f : 0;

    const T* a_col = BCAST ? a + bi * L : a + bi * L * F + fc;
    const int64_t a_stride = BCAST ? 1 : F;
    const T* b_col = b + bi * L * F + fc;
    T* h_col = h + bi * L * F + fc;

    A carry = col_ok ? static_cast<A>(h0[bi * F + fc]) : A(0);

    // Scan one chunk held in (ra, rb), starting at t0, and write its states.
    auto process = [&](A (&ra)[S], A (&rb)[S], int64_t t0) {
        const int64_t t_seg = t0 + static_cast<int64_t>(seg) * S;
        // Segment-local inclusive scan from a zero state: (prod a, local h).
        A p = A(1), q = A(0);
#pragma unroll
        for (int i = 0; i < S; ++i) {
            q = ra[i] * q + rb[i];
            p = p * ra[i];
            ra[i] = p;
            rb[i] = q;
        }
        seg_p[seg][lane] = p;
        seg_b[seg][lane] = q;
        __syncthreads();
        // Compose the carried state through the segments before this one.
        A c = carry, c_in = carry;
#pragma unroll
        for (int j = 0; j < NSEG; ++j) {
            if (j == seg) c_in = c;
            c = seg_p[j][lane] * c + seg_b[j][lane];
        }
        carry = c;
        if (col_ok) {
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const int64_t t = t_seg + i;
                if (t < L) h_col[t * F] = static_cast<T>(ra[i] * c_in + rb[i]);
            }
        }
        __syncthreads();
    };

    // Two register buffers, alternated by a two-chunk loop body, so that the
    // next chunk's loads are always in flight while the current one is scanned.
    A xa[S], xb[S], ya[S], yb[S];
    const int64_t seg_off = static_cast<int64_t>(seg) * S;
    scan_load<T, A, S, BCAST>(a_col, b_col, a_stride, F, L, seg_off, col_ok, xa, xb);
    for (int64_t t0 = 0; t0 < L; t0 += 2 * CH) {
        scan_load<T, A, S, BCAST>(a_col, b_col, a_stride, F, L, t0 + CH + seg_off, col_ok, ya, yb);
        process(xa, xb, t0);
        if (t0 + CH >= L) break;
        scan_load<T, A, S, BCAST>(a_col, b_col, a_stride, F, L, t0 + 2 * CH + seg_off, col_ok, xa, xb);
        process(ya, yb, t0 + CH);
    }
}

// fp32, full-shape retention, F % VEC == 0 and 16-byte aligned rows: each lane
// owns VEC adjacent columns (one VEC-wide vector load per step), so a wave
// reads 64 * VEC * 4 contiguous bytes of every step row. Same two-level
// structure and rounding as scan_forward_kernel (each column is scanned by the
// same operations in the same order).
template <int VEC>
struct FloatVec;
template <>
struct FloatVec<1> {
    using type = float;
    __device__ static void split(const float& v, float (&o)[1]) { o[0] = v; }
    __device__ static float join(const float (&o)[1]) { return o[0]; }
};
template <>
struct FloatVec<2> {
    using type = float2;
    __device__ static void split(const float2& v, float (&o)[2]) { o[0] = v.x; o[1] = v.y; }
    __device__ static float2 join(const float (&o)[2]) { return make_float2(o[0], o[1]); }
};
template <>
struct FloatVec<4> {
    using type = float4;
    __device__ static void split(const float4& v, float (&o)[4]) { o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w; }
    __device__ static float4 join(const float (&o)[4]) { return make_float4(o[0], o[1], o[2], o[3]); }
};


// Gate inputs of the fused gates + scan (GATES): a and b point at the two
// fp32 pre-activation products u W_r^T and u W_c^T (rows `stride` floats
// apart); the biases (null: none) and the valid bytes turn them into the gates
// of BoundedRecurrentState.gates (model/memory.py:22-26) with the masking of
// network.py:307-309, by the same expressions as the separate gate kernel
// (gates.hip).
struct GateInputs {
    const float* retention_bias;  // [F] or null
    const float* candidate_bias;  // [F] or null
    const uint8_t* valid;         // [B * L] or null
    __bf16* h16;                  // bf16 copy of the states, row (b, t) at (b L + t) h16_stride, or null
    int64_t h16_stride;           // elements between rows of h16 (F when contiguous)
};

// VEC bf16 values in one store (2 VEC bytes, aligned to it).
template <int VEC>
__device__ __forceinline__ void store_bf16(__bf16* dst, const float (&o)[VEC]) {
    if constexpr (VEC == 1) {
        dst[0] = static_cast<__bf16>(o[0]);
    } else {
        uint32_t u[VEC];
#pragma unroll
        for (int c = 0; c < VEC; ++c) u[c] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(o[c]));
        if constexpr (VEC == 2) {
            *reinterpret_cast<uint32_t*>(dst) = u[0] | (u[1] << 16);
        } else {
            static_assert(VEC == 4, "two or four columns per lane");
            *reinterpret_cast<uint2*>(dst) = make_uint2(u[0] | (u[1] << 16), u[2] | (u[3] << 16));
        }
    }
}

// One chunk's raw inputs of a wave: S steps of VEC columns and the steps'
// valid bytes, loaded unconditionally at clamped positions so that no branch
// waits on them; wide_gate turns them into (a, b) pairs when they are used.
// VEC consecutive pre-activations as loaded (fp32, or bf16: the GEMM's own
// output dtype) and their fp32 widening.
template <typename ZT, int VEC>
struct ZVec {
    using type = typename FloatVec<VEC>::type;
    __device__ static void split(const type& v, float (&o)[VEC]) { FloatVec<VEC>::split(v, o); }
};
template <int VEC>
struct ZVec<__bf16, VEC> {
    static_assert(VEC == 1 || VEC == 2 || VEC == 4, "one, two or four columns per lane");
    using type = std::conditional_t<VEC == 1, uint16_t, std::conditional_t<VEC == 2, uint32_t, uint2>>;
    __device__ static void split(const type& v, float (&o)[VEC]) {
        if constexpr (VEC == 1) {
            o[0] = __uint_as_float(static_cast<uint32_t>(v) << 16);
        } else if constexpr (VEC == 2) {
            o[0] = __uint_as_float(v << 16);
            o[1] = __uint_as_float(v & 0xffff0000u);
        } else {
            o[0] = __uint_as_float(v.x << 16);
            o[1] = __uint_as_float(v.x & 0xffff0000u);
            o[2] = __uint_as_float(v.y << 16);
            o[3] = __uint_as_float(v.y & 0xffff0000u);
        }
    }
};

template <int S, int VEC, typename ZT = float>
struct WideRaw {
    typename ZVec<ZT, VEC>::type va[S], vb[S];
    uint8_t keep[S];
};

template <int S, int VEC, bool GATES, typename ZT = float>
__device__ __forceinline__ void wide_fetch(const ZT* __restrict__ a_col, const ZT* __restrict__ b_col,
                                           int64_t stride, int64_t L, int64_t t_first, int64_t bi,
                                           const GateInputs& gates, WideRaw<S, VEC, ZT>& raw) {
    using V = typename ZVec<ZT, VEC>::type;
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const int64_t t = t_first + i;
        const int64_t tc = t < L ? t : L - 1;
        raw.va[i] = *reinterpret_cast<const V*>(a_col + tc * stride);
        raw.vb[i] = *reinterpret_cast<const V*>(b_col + tc * stride);
        if constexpr (GATES) raw.keep[i] = gates.valid == nullptr ? 1 : gates.valid[bi * L + tc];
    }
}

// (a, b) of the fetched steps: the gates first when GATES, then the identity
// (1, 0) outside the sequence or the columns.
template <int S, int VEC, bool GATES, typename ZT = float>
__device__ __forceinline__ void wide_gate(const WideRaw<S, VEC, ZT>& raw, int64_t L, int64_t t_first, bool col_ok,
                                          const float (&gbr)[VEC], const float (&gbc)[VEC], float (&ra)[S][VEC],
                                          float (&rb)[S][VEC]) {
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const bool ok = col_ok && t_first + i < L;
        ZVec<ZT, VEC>::split(raw.va[i], ra[i]);
        ZVec<ZT, VEC>::split(raw.vb[i], rb[i]);
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
            if constexpr (GATES) gate_pair(ra[i][c], rb[i][c], gbr[c], gbc[c], raw.keep[i] != 0, ra[i][c], rb[i][c]);
            ra[i][c] = ok ? ra[i][c] : 1.0f;
            rb[i][c] = ok ? rb[i][c] : 0.0f;
        }
    }
}

template <int VEC, bool GATES>
__device__ __forceinline__ void gate_biases(const GateInputs& gates, int64_t fc, float (&gbr)[VEC],
                                            float (&gbc)[VEC]) {
    using V = typename FloatVec<VEC>::type;
#pragma unroll
    for (int c = 0; c < VEC; ++c) gbr[c] = gbc[c] = 0.0f;
    if constexpr (GATES) {
        if (gates.retention_bias) FloatVec<VEC>::split(*reinterpret_cast<const V*>(gates.retention_bias + fc), gbr);
        if (gates.candidate_bias) FloatVec<VEC>::split(*reinterpret_cast<const V*>(gates.candidate_bias + fc), gbc);
    }
}

// Two-phase scan, phase one: the transfer (P, Q) = (prod a, scan from 0) of
// every S-step segment j (positions j S .. j S + S - 1) of every column, by the
// operations of the segment pass of scan_forward_wide_kernel in their order,
// into tp / tq [B, segments, F]. Wave w of workgroup (x, y) takes segment
// 8 y + w of batch row x / col_tiles.
template <int S, int VEC, bool GATES, typename ZT = float>
__global__ __launch_bounds__(kWave * 8) void scan_segment_transfer_kernel(
    const ZT* __restrict__ a, const ZT* __restrict__ b, float* __restrict__ tp, float* __restrict__ tq,
    int64_t L, int64_t F, int64_t col_tiles, int64_t stride, int64_t segments, GateInputs gates) {
    using V = typename FloatVec<VEC>::type;
    const int lane = lane_id();
    const int64_t j = static_cast<int64_t>(blockIdx.y) * 8 + static_cast<int>(threadIdx.x) / kWave;
    if (j >= segments) return;
    const int64_t bi = static_cast<int64_t>(blockIdx.x) / col_tiles;
    const int64_t f = ((static_cast<int64_t>(blockIdx.x) % col_tiles) * kWave + lane) * VEC;
    const bool col_ok = f < F;
    const int64_t fc = col_ok ? f : 0;
    float gbr[VEC], gbc[VEC];
    gate_biases<VEC, GATES>(gates, fc, gbr, gbc);
    WideRaw<S, VEC, ZT> raw;
    wide_fetch<S, VEC, GATES, ZT>(a + bi * L * stride + fc, b + bi * L * stride + fc, stride, L, j * S, bi, gates,
                                  raw);
    float ra[S][VEC], rb[S][VEC];
    wide_gate<S, VEC, GATES, ZT>(raw, L, j * S, col_ok, gbr, gbc, ra, rb);
    float po[VEC], qo[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
        float p = 1.0f, q = 0.0f;
#pragma unroll
        for (int i = 0; i < S; ++i) {
            q = ra[i][c] * q + rb[i][c];
            p = p * ra[i][c];
        }
        po[c] = p;
        qo[c] = q;
    }
    if (col_ok) {
        const int64_t o = (bi * segments + j) * F + f;
        *reinterpret_cast<V*>(tp + o) = FloatVec<VEC>::join(po);
        *reinterpret_cast<V*>(tq + o) = FloatVec<VEC>::join(qo);
    }
}

// Two-phase scan, between the phases: the carried state at the start of every
// chunk of `spc` segments, c <- P_j c + Q_j over the segments in order from
// h0, into carries [B, chunks, F] (chunk 0's is h0 itself and is not written).
// One workgroup per 64 columns of a batch row: in each round of 256 segments,
// wave w first loads the transfers of segments 32 w .. 32 w + 31 (all loads in
// flight together), then the waves fold their segments one after the other,
// handing the carry on through LDS.
constexpr int kCarrySegs = 32;
__global__ __launch_bounds__(kWave * 8) void scan_chunk_carry_kernel(
    const float* __restrict__ tp, const float* __restrict__ tq, const float* __restrict__ h0,
    float* __restrict__ carries, int64_t F, int64_t col_tiles, int64_t segments, int64_t spc, int64_t chunks) {
    __shared__ float hand[kWave];
    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int64_t bi = static_cast<int64_t>(blockIdx.x) / col_tiles;
    const int64_t f = (static_cast<int64_t>(blockIdx.x) % col_tiles) * kWave + lane;
    const bool col_ok = f < F;
    const int64_t fc = col_ok ? f : 0;
    const float* tp_col = tp + bi * segments * F + fc;
    const float* tq_col = tq + bi * segments * F + fc;
    float carry = h0[bi * F + fc];
    for (int64_t r0 = 0; r0 < segments; r0 += 8 * kCarrySegs) {
        const int64_t j0 = r0 + static_cast<int64_t>(wave) * kCarrySegs;
        float p[kCarrySegs], q[kCarrySegs];
#pragma unroll
        for (int i = 0; i < kCarrySegs; ++i) {
            const int64_t j = j0 + i < segments ? j0 + i : segments - 1;
            p[i] = tp_col[j * F];
            q[i] = tq_col[j * F];
        }
        for (int w = 0; w < 8; ++w) {
            if (wave == w) {
                if (r0 > 0 || w > 0) carry = hand[lane];
                // the next chunk start at or after j0 + 1 (chunk starts are multiples of spc)
                int64_t next = (j0 / spc + 1) * spc;
                int64_t chunk = next / spc;
#pragma unroll
                for (int i = 0; i < kCarrySegs; ++i) {
                    const int64_t j = j0 + i;
                    if (j < segments) {
                        carry = p[i] * carry + q[i];
                        if (j + 1 == next) {
                            if (chunk < chunks && col_ok) carries[(bi * chunks + chunk) * F + f] = carry;
                            next += spc;
                            ++chunk;
                        }
                    }
                }
                hand[lane] = carry;
            }
            __syncthreads();
        }
    }
}

// The scan proper. Without chunk carries one workgroup walks its columns
// through the whole sequence. With them (phase two of the two-phase scan)
// workgroup (x, y) walks positions [y span, min(L, (y + 1) span)), span a
// multiple of NSEG * S, from chunk y's carry (h0 for y = 0): that carry is the
// state the one-workgroup walk carries into position y span, composed by the
// same operations in the same order, so both give the same bits.
//
// LPC > 1 splits each wave into LPC groups of 64 / LPC lanes: a workgroup then
// owns 64 / LPC column strips and NSEG * LPC segments per chunk (twice the
// workgroups for a batch of few rows at LPC = 2). The composition order, and
// so every result bit, is the same for any LPC and VEC.
//
// NTS: the states are written with non-temporal stores (outputs written once
// and far larger than the caches).
template <int S, int NSEG, int VEC, bool GATES = false, int LPC = 1, typename ZT = float, bool NTS = false>
__global__ __launch_bounds__(kWave * NSEG) void scan_forward_wide_kernel(
    const ZT* __restrict__ a, const ZT* __restrict__ b, const float* __restrict__ h0, float* __restrict__ h,
    int64_t L, int64_t F, int64_t col_tiles, int64_t stride,
    GateInputs gates = GateInputs{nullptr, nullptr, nullptr, nullptr, 0},
    const float* __restrict__ chunk_carry = nullptr, int64_t chunks = 0, int64_t span = 0) {
    using V = typename FloatVec<VEC>::type;
    constexpr int TW = kWave / LPC;    // lanes (column strips) per group
    constexpr int NS = NSEG * LPC;     // segments per chunk
    constexpr int CH = S * NS;
    __shared__ float seg_p[NS][VEC][TW];
    __shared__ float seg_b[NS][VEC][TW];

    const int lane = lane_id() % TW;
    const int seg = static_cast<int>(threadIdx.x) / kWave * LPC + lane_id() / TW;
    const int64_t bi = static_cast<int64_t>(blockIdx.x) / col_tiles;
    const int64_t f = ((static_cast<int64_t>(blockIdx.x) % col_tiles) * TW + lane) * VEC;
    const bool col_ok = f < F;
    const int64_t fc = col_ok ? f : 0;
    const ZT* a_col = a + bi * L * stride + fc;
    const ZT* b_col = b + bi * L * stride + fc;
    float* h_col = h + bi * L * F + fc;
    const int64_t t_begin = chunk_carry != nullptr ? static_cast<int64_t>(blockIdx.y) * span : 0;
    const int64_t t_end = chunk_carry != nullptr ? (t_begin + span < L ? t_begin + span : L) : L;

    float gbr[VEC], gbc[VEC];
    gate_biases<VEC, GATES>(gates, fc, gbr, gbc);
    float carry[VEC];
    {
        const V c0 = *reinterpret_cast<const V*>(h0 + bi * F + fc);
        FloatVec<VEC>::split(c0, carry);
#pragma unroll
        for (int c = 0; c < VEC; ++c) carry[c] = col_ok ? carry[c] : 0.0f;
    }
    if (chunk_carry != nullptr && blockIdx.y > 0) {
        const V cy = *reinterpret_cast<const V*>(chunk_carry + (bi * chunks + blockIdx.y) * F + fc);
        FloatVec<VEC>::split(cy, carry);
#pragma unroll
        for (int c = 0; c < VEC; ++c) carry[c] = col_ok ? carry[c] : 0.0f;
    }

    auto fetch = [&](int64_t t_first, WideRaw<S, VEC, ZT>& raw) {
        wide_fetch<S, VEC, GATES, ZT>(a_col, b_col, stride, L, t_first, bi, gates, raw);
    };

    auto process = [&](float (&ra)[S][VEC], float (&rb)[S][VEC], int64_t t0) {
        const int64_t t_seg = t0 + static_cast<int64_t>(seg) * S;
        float c_in[VEC];
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
            float p = 1.0f, q = 0.0f;
#pragma unroll
            for (int i = 0; i < S; ++i) {
                q = ra[i][c] * q + rb[i][c];
                p = p * ra[i][c];
                ra[i][c] = p;
                rb[i][c] = q;
            }
            seg_p[seg][c][lane] = p;
            seg_b[seg][c][lane] = q;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < VEC; ++c) {
            float cc = carry[c], ci = carry[c];
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                if (j == seg) ci = cc;
                cc = seg_p[j][c][lane] * cc + seg_b[j][c][lane];
            }
            carry[c] = cc;
            c_in[c] = ci;
        }
        if (col_ok) {
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const int64_t t = t_seg + i;
                float o[VEC];
#pragma unroll
                for (int c = 0; c < VEC; ++c) o[c] = ra[i][c] * c_in[c] + rb[i][c];
                if (t < t_end) {
                    if constexpr (NTS) {
                        typedef float f32xv __attribute__((ext_vector_type(VEC)));
                        f32xv ov;
#pragma unroll
                        for (int c = 0; c < VEC; ++c) ov[c] = o[c];
                        __builtin_nontemporal_store(ov, reinterpret_cast<f32xv*>(h_col + t * F));
                    } else {
                        *reinterpret_cast<V*>(h_col + t * F) = FloatVec<VEC>::join(o);
                    }
                    if constexpr (GATES) {
                        if (gates.h16 != nullptr) store_bf16<VEC>(gates.h16 + (bi * L + t) * gates.h16_stride + f, o);
                    }
                }
            }
        }
        __syncthreads();
    };

    // A ring of NB chunk buffers: the loads of the next NB - 1 chunks are in
    // flight while one is scanned (buffer indices are compile-time constants
    // of the unrolled ring, so the buffers stay in registers).
    constexpr int NB = VEC == 1 ? KOEMI_SCAN_BUFFERS : 2;
    WideRaw<S, VEC, ZT> raw[NB];
    const int64_t seg_off = static_cast<int64_t>(seg) * S;
#pragma unroll
    for (int k = 0; k + 1 < NB; ++k) fetch(t_begin + k * CH + seg_off, raw[k]);
    for (int64_t t0 = t_begin; t0 < t_end; t0 += NB * CH) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int64_t tc = t0 + k * CH;
            if (tc >= t_end) break;
            fetch(tc + (NB - 1) * CH + seg_off, raw[(k + NB - 1) % NB]);
            float ra[S][VEC], rb[S][VEC];
            wide_gate<S, VEC, GATES, ZT>(raw[k], L, tc + seg_off, col_ok, gbr, gbc, ra, rb);
            process(ra, rb, tc);
        }
    }
}

// Reverse-time adjoint of the scan (dense/affine_scan.cu:58-106):
//   g_t = dh_t + a_{t+1} g_{t+1},  db_t = g_t,  da_t = g_t h_{t-1},  dh0 = a_0 g_0.
// In reversed time u = L-1-t this is a forward scan with coefficient a_{t+1}
// and increment dh_t, so it reuses the same two-level structure.
template <typename T, int S, int NSEG, bool BCAST>
__global__ __launch_bounds__(kWave * NSEG) void scan_backward_kernel(
    const T* __restrict__ a, const T* __restrict__ h0, const T* __restrict__ h,
    const T* __restrict__ dh, T* __restrict__ da, T* __restrict__ db, T* __restrict__ dh0,
    int64_t L, int64_t F, int64_t col_tiles) {
    using A = typename AccOf<T>::type;
    constexpr int CH = S * NSEG;
    __shared__ A seg_p[NSEG][kWave];
    __shared__ A seg_b[NSEG][kWave];

    const int lane = lane_id();
    const int seg = static_cast<int>(threadIdx.x) / kWave;
    const int64_t bi = static_cast<int64_t>(blockIdx.x) / col_tiles;
    const int64_t f = (static_cast<int64_t>(blockIdx.x) % col_tiles) * kWave + lane;
    const bool col_ok = f < F;
    const int64_t fc = col_ok ? f : 0;

    const T* a_col = BCAST ? a + bi * L : a + bi * L * F + fc;
    const int64_t a_stride = BCAST ? 1 : F;
    const int64_t base = bi * L * F + fc;
    const A h_init = col_ok ? static_cast<A>(h0[bi * F + fc]) : A(0);

    A carry = A(0);
    for (int64_t u0 = 0; u0 < L; u0 += CH) {
        const int64_t u_seg = u0 + static_cast<int64_t>(seg) * S;
        A ra[S], rb[S], hp[S];
        T va[S], vg[S], vh[S];
#pragma unroll
        for (int i = 0; i < S; ++i) {  // unconditional, clamped loads (see scan_load)
            const int64_t t = L - 1 - (u_seg + i);
            const int64_t tc = t < 0 ? 0 : t;
            const int64_t ta = tc + 1 < L ? tc + 1 : L - 1;
            const int64_t tp = tc > 0 ? tc - 1 : 0;
            va[i] = a_col[ta * a_stride];
            vg[i] = dh[base + tc * F];
            vh[i] = h[base + tp * F];
        }
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const int64_t t = L - 1 - (u_seg + i);
            const bool ok = col_ok && t >= 0;
            ra[i] = (ok && t + 1 < L) ? static_cast<A>(va[i]) : A(1);
            rb[i] = ok ? static_cast<A>(vg[i]) : A(0);
            hp[i] = ok ? (t > 0 ? static_cast<A>(vh[i]) : h_init) : A(0);
        }
        A p = A(1), q = A(0);
#pragma unroll
        for (int i = 0; i < S; ++i) {
            q = ra[i] * q + rb[i];
            p = p * ra[i];
            ra[i] = p;
            rb[i] = q;
        }
        seg_p[seg][lane] = p;
        seg_b[seg][lane] = q;
        __syncthreads();
        A c = carry, c_in = carry;
#pragma unroll
        for (int j = 0; j < NSEG; ++j) {
            if (j == seg) c_in = c;
            c = seg_p[j][lane] * c + seg_b[j][lane];
        }
        carry = c;
        if (col_ok) {
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const int64_t t = L - 1 - (u_seg + i);
                if (t >= 0) {
                    const A g = ra[i] * c_in + rb[i];
                    db[base + t * F] = static_cast<T>(g);
                    da[base + t * F] = static_cast<T>(g * hp[i]);
                }
            }
        }
        __syncthreads();
    }
    if (col_ok && seg == 0) {
        dh0[bi * F + fc] = static_cast<T>(static_cast<A>(a_col[0]) * carry);
    }
}

#ifndef KOEMI_SCAN_VEC
#define KOEMI_SCAN_VEC 2
#endif

template <typename T, bool BCAST>
int launch_forward(const void* a, const void* b, const void* h0, void* h, int64_t B, int64_t L,
                   int64_t F, hipStream_t stream) {
    if constexpr (std::is_same<T, float>::value && !BCAST && KOEMI_SCAN_VEC > 1) {
        constexpr int VEC = KOEMI_SCAN_VEC;
        const bool wide = F % VEC == 0 && reinterpret_cast<uintptr_t>(a) % (4 * VEC) == 0 &&
                          reinterpret_cast<uintptr_t>(b) % (4 * VEC) == 0 &&
                          reinterpret_cast<uintptr_t>(h) % (4 * VEC) == 0 &&
                          reinterpret_cast<uintptr_t>(h0) % (4 * VEC) == 0;
        const int64_t tiles = (F / VEC + kWave - 1) / kWave;
        // Wider column strips halve the workgroup count; keep at least one per CU.
        if (wide && B * tiles >= 256) {
            const int64_t blocks = B * tiles;
            if (blocks > 0x7fffffff) return fail(KOEMI_ERR_UNSUPPORTED, "affine scan grid too large");
            auto launch = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kWave * kScanSegments), 0,
                                   stream, static_cast<const float*>(a), static_cast<const float*>(b),
                                   static_cast<const float*>(h0), static_cast<float*>(h), L, F, tiles, F,
                                   GateInputs{nullptr, nullptr, nullptr, nullptr, 0}, nullptr, 0, 0);
            };
            if (B * L * F * 4 > KOEMI_NT_STORE_BYTES)  // measured at C3: 278 -> 270 us
                launch(scan_forward_wide_kernel<kScanSteps, kScanSegments, VEC, false, 1, float, true>);
            else
                launch(scan_forward_wide_kernel<kScanSteps, kScanSegments, VEC>);
            return check_launch("koemi_affine_scan_forward");
        }
    }
    const int64_t col_tiles = (F + kWave - 1) / kWave;
    const int64_t blocks = B * col_tiles;
    if (blocks > 0x7fffffff) return fail(KOEMI_ERR_UNSUPPORTED, "affine scan grid too large");
    hipLaunchKernelGGL((scan_forward_kernel<T, kScanSteps, kScanSegments, BCAST>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kWave * kScanSegments), 0, stream,
                       static_cast<const T*>(a), static_cast<const T*>(b),
                       static_cast<const T*>(h0), static_cast<T*>(h), L, F, col_tiles);
    return check_launch("koemi_affine_scan_forward");
}

template <typename T, bool BCAST>
int launch_backward(const void* a, const void* h0, const void* h, const void* dh, void* da,
                    void* db, void* dh0, int64_t B, int64_t L, int64_t F, hipStream_t stream) {
    const int64_t col_tiles = (F + kWave - 1) / kWave;
    const int64_t blocks = B * col_tiles;
    if (blocks > 0x7fffffff) return fail(KOEMI_ERR_UNSUPPORTED, "affine scan grid too large");
    hipLaunchKernelGGL((scan_backward_kernel<T, kScanSteps, kScanSegments, BCAST>),
                       dim3(static_cast<unsigned>(blocks)), dim3(kWave * kScanSegments), 0, stream,
                       static_cast<const T*>(a), static_cast<const T*>(h0),
                       static_cast<const T*>(h), static_cast<const T*>(dh), static_cast<T*>(da),
                       static_cast<T*>(db), static_cast<T*>(dh0), L, F, col_tiles);
    return check_launch("koemi_affine_scan_backward");
}

int check_scan_args(const void* a, const void* b, const void* h0, const void* h, int64_t B,
                    int64_t L, int64_t F, int dtype) {
    if (B < 0 || L < 0 || F < 0) return fail(KOEMI_ERR_INVALID, "affine scan sizes must be non-negative");
    if (dtype != KOEMI_F32 && dtype != KOEMI_F64 && dtype != KOEMI_F16 && dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "affine scan does not support dtype %s", dtype_name(dtype));
    if (B * L * F > 0 && (!a || !b || !h0 || !h))
        return fail(KOEMI_ERR_INVALID, "affine scan received a null pointer");
    return KOEMI_OK;
}

}  // namespace

// One-position windows (decode steps): h = a h0 + b per column, the same
// single rounding the scan makes at its first position.
template <typename ZT>
__global__ __launch_bounds__(256) void gated_step_kernel(const ZT* __restrict__ zr, const ZT* __restrict__ zc,
                                                         int64_t stride, GateInputs gates,
                                                         const float* __restrict__ h0, float* __restrict__ h,
                                                         int64_t B, int64_t F) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= B * F) return;
    const int64_t bi = i / F, f = i - bi * F;
    const bool keep = gates.valid == nullptr || gates.valid[bi] != 0;
    float a, b;
    gate_pair(to_f32(zr[bi * stride + f]), to_f32(zc[bi * stride + f]),
              gates.retention_bias ? gates.retention_bias[f] : 0.0f,
              gates.candidate_bias ? gates.candidate_bias[f] : 0.0f, keep, a, b);
    const float hv = a * h0[i] + b;
    h[i] = hv;
    if (gates.h16 != nullptr) gates.h16[bi * gates.h16_stride + f] = static_cast<__bf16>(hv);
}

// Two-phase split of an S-step segmented walk over L positions into chunks of
// `span` positions (a multiple of NSEG * S): enough chunks that about
// kTwoPhaseBlocks workgroups run (none when the column tiles alone fill that
// many, or the sequence is a single chunk).
constexpr int64_t kTwoPhaseBlocks = 1024;
struct TwoPhase {
    int64_t span = 0, chunks = 0, segments = 0;
};
inline TwoPhase two_phase_split(int64_t col_blocks, int64_t L) {
    constexpr int64_t CH = static_cast<int64_t>(kScanSteps) * kScanSegments;
    TwoPhase tp;
    const int64_t steps = (L + CH - 1) / CH;
    int64_t want = (kTwoPhaseBlocks + col_blocks - 1) / col_blocks;
    if (want > steps) want = steps;
    if (want < 2) return tp;
    tp.span = (steps + want - 1) / want * CH;
    tp.chunks = (L + tp.span - 1) / tp.span;
    tp.segments = (L + kScanSteps - 1) / kScanSteps;
    if (tp.chunks < 2 || tp.chunks > 65535 || (tp.segments + 7) / 8 > 65535) tp.chunks = 0;
    return tp;
}

// Workspace of the two-phase scan: the segment transfers P and Q, then the
// chunk carries (at most one chunk per NSEG * S positions).
size_t gated_scan_workspace(int64_t B, int64_t L, int64_t F) {
    constexpr int64_t CH = static_cast<int64_t>(kScanSteps) * kScanSegments;
    const size_t segments = static_cast<size_t>((L + kScanSteps - 1) / kScanSteps);
    const size_t chunks = static_cast<size_t>((L + CH - 1) / CH);
    return (2 * segments + chunks) * static_cast<size_t>(B) * static_cast<size_t>(F) * sizeof(float);
}

#ifndef KOEMI_SCAN_TWO_PHASE_VEC
#define KOEMI_SCAN_TWO_PHASE_VEC 2
#endif
#ifndef KOEMI_SCAN_LPC_MAX
#define KOEMI_SCAN_LPC_MAX 2
#endif
#ifndef KOEMI_SCAN_TWO_PHASE_BELOW
#define KOEMI_SCAN_TWO_PHASE_BELOW 128
#endif
// The one-pass scan runs when it has at least this many workgroups.
constexpr int64_t kTwoPhaseBelow = KOEMI_SCAN_TWO_PHASE_BELOW;

// The three launches of the two-phase gated scan, VEC columns per lane in the
// two passes over the pre-activations (the carry pass works column by column
// on the [B, segments, F] transfers, whatever VEC is).
template <int VEC, typename ZT>
int run_two_phase(const ZT* zr, const ZT* zc, int64_t stride, const GateInputs& gates, const float* h0, float* h,
                  int64_t B, int64_t L, int64_t F, int64_t tiles, const TwoPhase& split, float* workspace,
                  hipStream_t stream) {
    float* tp = workspace;
    float* tq = tp + B * split.segments * F;
    float* carries = tq + B * split.segments * F;
    hipLaunchKernelGGL((scan_segment_transfer_kernel<kScanSteps, VEC, true, ZT>),
                       dim3(static_cast<unsigned>(B * tiles), static_cast<unsigned>((split.segments + 7) / 8)),
                       dim3(kWave * 8), 0, stream, zr, zc, tp, tq, L, F, tiles, stride, split.segments, gates);
    int st = check_launch("gated scan (segment transfers)");
    if (st != KOEMI_OK) return st;
    const int64_t carry_tiles = (F + kWave - 1) / kWave;
    hipLaunchKernelGGL(scan_chunk_carry_kernel, dim3(static_cast<unsigned>(B * carry_tiles)), dim3(kWave * 8), 0,
                       stream, tp, tq, h0, carries, F, carry_tiles, split.segments, split.span / kScanSteps,
                       split.chunks);
    st = check_launch("gated scan (chunk carries)");
    if (st != KOEMI_OK) return st;
    hipLaunchKernelGGL((scan_forward_wide_kernel<kScanSteps, kScanSegments, VEC, true, 1, ZT>),
                       dim3(static_cast<unsigned>(B * tiles), static_cast<unsigned>(split.chunks)),
                       dim3(kWave * kScanSegments), 0, stream, zr, zc, h0, h, L, F, tiles, stride, gates, carries,
                       split.chunks, split.span);
    return check_launch("gated scan (chunks)");
}

// The fused gates + scan over fp32 pre-activation products zr, zc (row r of
// the B x L rows at r * stride): one position per column for L == 1,
// otherwise the wide scan with KOEMI_SCAN_VEC columns per lane where the rows
// are aligned to it and that still fills the chip; one column per lane
// otherwise, split into the two-phase scan (segment transfers into the
// workspace, then chunks of the sequence walked from their carried state) when
// a workspace of gated_scan_workspace bytes is given and the column tiles
// alone leave the chip short of workgroups. The caller has checked that
// B * ceil(F / 64) fits the grid.
template <typename ZT>
int launch_gated_scan_t(const ZT* zr, const ZT* zc, int64_t stride, const float* retention_bias,
                        const float* candidate_bias, const uint8_t* valid, const float* h0, float* h, void* h16,
                        int64_t h16_stride, int64_t B, int64_t L, int64_t F, hipStream_t stream, void* workspace,
                        size_t workspace_bytes) {
    constexpr int VEC = KOEMI_SCAN_VEC;
    const GateInputs gates{retention_bias, candidate_bias, valid, static_cast<__bf16*>(h16), h16_stride};
    if (L == 1) {
        hipLaunchKernelGGL(gated_step_kernel<ZT>, dim3(static_cast<unsigned>((B * F + 255) / 256)), dim3(256), 0, stream,
                           zr, zc, stride, gates, h0, h, B, F);
        return check_launch("gated scan (one position)");
    }
    auto aligned = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % (4 * VEC) == 0; };
    const int64_t wide_tiles = (F / VEC + kWave - 1) / kWave;
    if (F % VEC == 0 && stride % VEC == 0 && aligned(zr) && aligned(zc) && aligned(h) && aligned(h0) &&
        aligned(retention_bias) && aligned(candidate_bias) && reinterpret_cast<uintptr_t>(h16) % (2 * VEC) == 0 &&
        h16_stride % VEC == 0 &&
        B * wide_tiles >= 256) {
        hipLaunchKernelGGL((scan_forward_wide_kernel<kScanSteps, kScanSegments, VEC, true, 1, ZT>),
                           dim3(static_cast<unsigned>(B * wide_tiles)), dim3(kWave * kScanSegments), 0, stream, zr, zc,
                           h0, h, L, F, wide_tiles, stride, gates);
        return check_launch("gated scan");
    }
    // One column per lane: lane groups of 64 / lpc lanes, lpc = 2 or 4 when
    // the batch's 64-column strips leave CUs idle.
    int lpc = 1;
    while (lpc < KOEMI_SCAN_LPC_MAX && B * ((F + kWave / lpc - 1) / (kWave / lpc)) < 256 && F > kWave / lpc / 2)
        lpc *= 2;
    const int64_t tiles = (F + kWave / lpc - 1) / (kWave / lpc);
    if (workspace != nullptr && workspace_bytes >= gated_scan_workspace(B, L, F) && B * tiles < kTwoPhaseBelow) {
        constexpr int TV = KOEMI_SCAN_TWO_PHASE_VEC;
        const bool tv_ok = F % TV == 0 && stride % TV == 0 && reinterpret_cast<uintptr_t>(workspace) % (4 * TV) == 0 &&
                           reinterpret_cast<uintptr_t>(h16) % (2 * TV) == 0 && h16_stride % TV == 0 &&
                           [&] {
                               for (const void* p : {static_cast<const void*>(zr), static_cast<const void*>(zc),
                                                     static_cast<const void*>(h), static_cast<const void*>(h0),
                                                     static_cast<const void*>(retention_bias),
                                                     static_cast<const void*>(candidate_bias)})
                                   if (p != nullptr && reinterpret_cast<uintptr_t>(p) % (4 * TV) != 0) return false;
                               return true;
                           }();
        const int64_t tiles1 = (F + kWave - 1) / kWave;
        const int64_t tv_tiles = (F / TV + kWave - 1) / kWave;
        const TwoPhase split = two_phase_split(B * (tv_ok ? tv_tiles : tiles1), L);
        if (split.chunks >= 2) {
            if (tv_ok)
                return run_two_phase<TV, ZT>(zr, zc, stride, gates, h0, h, B, L, F, tv_tiles, split,
                                             static_cast<float*>(workspace), stream);
            return run_two_phase<1, ZT>(zr, zc, stride, gates, h0, h, B, L, F, tiles1, split,
                                        static_cast<float*>(workspace), stream);
        }
    }
    auto one_pass = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(B * tiles)), dim3(kWave * kScanSegments), 0, stream, zr,
                           zc, h0, h, L, F, tiles, stride, gates, nullptr, 0, 0);
    };
    if (lpc == 4) one_pass(scan_forward_wide_kernel<kScanSteps, kScanSegments, 1, true, 4, ZT>);
    else if (lpc == 2) one_pass(scan_forward_wide_kernel<kScanSteps, kScanSegments, 1, true, 2, ZT>);
    else one_pass(scan_forward_wide_kernel<kScanSteps, kScanSegments, 1, true, 1, ZT>);
    return check_launch("gated scan");
}

int launch_gated_scan(const float* zr, const float* zc, int64_t stride, const float* retention_bias,
                      const float* candidate_bias, const uint8_t* valid, const float* h0, float* h, void* h16,
                      int64_t h16_stride, int64_t B, int64_t L, int64_t F, hipStream_t stream, void* workspace,
                      size_t workspace_bytes) {
    return launch_gated_scan_t(zr, zc, stride, retention_bias, candidate_bias, valid, h0, h, h16, h16_stride, B, L,
                               F, stream, workspace, workspace_bytes);
}

}  // namespace koemi

using namespace koemi;

extern "C" int koemi_affine_scan_forward(const void* retention, const void* increment,
                                         const void* initial, void* states, int64_t batch,
                                         int64_t sequence, int64_t features,
                                         int broadcast_retention, int dtype,
                                         koemi_stream_t stream) {
    int st = check_scan_args(retention, increment, initial, states, batch, sequence, features, dtype);
    if (st != KOEMI_OK) return st;
    if (batch * sequence * features == 0) return KOEMI_OK;
    hipStream_t s = as_stream(stream);
    const bool bc = broadcast_retention != 0;
    switch (dtype) {
        case KOEMI_F32:
            return bc ? launch_forward<float, true>(retention, increment, initial, states, batch, sequence, features, s)
                      : launch_forward<float, false>(retention, increment, initial, states, batch, sequence, features, s);
        case KOEMI_F64:
            return bc ? launch_forward<double, true>(retention, increment, initial, states, batch, sequence, features, s)
                      : launch_forward<double, false>(retention, increment, initial, states, batch, sequence, features, s);
        case KOEMI_F16:
            return bc ? launch_forward<f16, true>(retention, increment, initial, states, batch, sequence, features, s)
                      : launch_forward<f16, false>(retention, increment, initial, states, batch, sequence, features, s);
        default:
            return bc ? launch_forward<bf16, true>(retention, increment, initial, states, batch, sequence, features, s)
                      : launch_forward<bf16, false>(retention, increment, initial, states, batch, sequence, features, s);
    }
}

extern "C" int koemi_affine_scan_backward(const void* retention, const void* initial,
                                          const void* states, const void* grad_states,
                                          void* grad_retention, void* grad_increment,
                                          void* grad_initial, int64_t batch, int64_t sequence,
                                          int64_t features, int broadcast_retention, int dtype,
                                          koemi_stream_t stream) {
    int st = check_scan_args(retention, states, initial, grad_states, batch, sequence, features, dtype);
    if (st != KOEMI_OK) return st;
    if (batch * sequence * features > 0 && (!grad_retention || !grad_increment || !grad_initial))
        return fail(KOEMI_ERR_INVALID, "affine scan backward received a null gradient pointer");
    if (batch * sequence * features == 0) return KOEMI_OK;
    hipStream_t s = as_stream(stream);
    const bool bc = broadcast_retention != 0;
#define KOEMI_SCAN_BWD(T)                                                                          \
    (bc ? launch_backward<T, true>(retention, initial, states, grad_states, grad_retention,        \
                                   grad_increment, grad_initial, batch, sequence, features, s)    \
        : launch_backward<T, false>(retention, initial, states, grad_states, grad_retention,       \
                                    grad_increment, grad_initial, batch, sequence, features, s))
    switch (dtype) {
        case KOEMI_F32: return KOEMI_SCAN_BWD(float);
        case KOEMI_F64: return KOEMI_SCAN_BWD(double);
        case KOEMI_F16: return KOEMI_SCAN_BWD(f16);
        default: return KOEMI_SCAN_BWD(bf16);
    }
#undef KOEMI_SCAN_BWD
}

extern "C" size_t koemi_gated_scan_workspace_bytes(int64_t batch, int64_t length, int64_t width) {
    if (batch <= 0 || length <= 1 || width <= 0) return 0;
    return gated_scan_workspace(batch, length, width);
}

extern "C" int koemi_gated_scan(const void* preactivations, int preactivation_dtype, int64_t row_stride,
                                int64_t retention_offset, int64_t candidate_offset, const float* retention_bias,
                                const float* candidate_bias, const uint8_t* valid, const float* initial, float* states,
                                void* states_bf16, int64_t bf16_row_stride, int64_t batch, int64_t length,
                                int64_t width, void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "gated scan needs non-negative batch and length and a positive width");
    if (preactivation_dtype != KOEMI_F32 && preactivation_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "gated scan pre-activations must be float32 or bfloat16");
    if (retention_offset < 0 || candidate_offset < 0 || retention_offset + width > row_stride ||
        candidate_offset + width > row_stride)
        return fail(KOEMI_ERR_INVALID, "gated scan: the gate columns must lie inside a row");
    if (batch * length == 0) return KOEMI_OK;
    if (!preactivations || !initial || !states) return fail(KOEMI_ERR_INVALID, "gated scan received a null pointer");
    if (batch * ((width + kWave - 1) / kWave) > 0x7fffffffLL || batch * width > 0x7fffffffLL * 256LL)
        return fail(KOEMI_ERR_UNSUPPORTED, "gated scan grid too large");
    if (bf16_row_stride == 0) bf16_row_stride = width;
    if (states_bf16 != nullptr && bf16_row_stride < width)
        return fail(KOEMI_ERR_INVALID, "gated scan: the bf16 row stride is below the width");
    if (workspace != nullptr && workspace_bytes < gated_scan_workspace(batch, length, width))
        return fail(KOEMI_ERR_INVALID, "gated scan workspace too small: need %zu bytes",
                    gated_scan_workspace(batch, length, width));
    if (preactivation_dtype == KOEMI_BF16) {
        const bf16* z = static_cast<const bf16*>(preactivations);
        return launch_gated_scan_t(z + retention_offset, z + candidate_offset, row_stride, retention_bias,
                                   candidate_bias, valid, initial, states, states_bf16, bf16_row_stride, batch, length,
                                   width, as_stream(stream), workspace, workspace_bytes);
    }
    const float* z = static_cast<const float*>(preactivations);
    return launch_gated_scan_t(z + retention_offset, z + candidate_offset, row_stride, retention_bias, candidate_bias,
                               valid, initial, states, states_bf16, bf16_row_stride, batch, length, width,
                               as_stream(stream), workspace, workspace_bytes);
}
