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
// Up to kFusedMaxSlots slots (S + L) three HIP kernels, products on fp32 MFMA
// (v_mfma_f32_32x32x2f32) with every operand converted to fp32 and loaded
// straight from memory into the MFMA operand registers (no LDS staging):
//   scores: one workgroup per active (32 slots, 32 queries, batch, quarter of
//     the width) tile, a tile being active when some slot in it is eligible
//     for some query of it; four fp32 partial score arrays.
//   softmax: one wave per query row; adds the partials, masks, max, exp, sum
//     in registers, writes fp32 weights (zero rows when nothing is eligible).
//   weighted sum: one workgroup per (128 output columns, 32 queries, batch),
//     slot blocks past the tile's last eligible slot skipped.
// The local memory's read (LocalKeyValueMemory.read_window, memory.py:332-362)
// is the same masked read with a sliding window: slot s is eligible for query t
// when its valid byte is set and S + t - window <= s < S + t (the window
// entries strictly before the query's own entry; memory.py:364-383).
//
// Longer slot axes use rocBLAS for the two products (fp32 accumulation; the
// carried and window parts of the key axis as separate strided-batched calls
// on the caller's tensors) around a masked-softmax kernel. rocBLAS is
// column-major: a row-major [rows, cols] matrix is its [cols, rows]
// column-major view, so score^T = K'^T Q' and out' = V' P'.
#include "common.hpp"
#include "step_memory.hpp"

#include <rocblas/rocblas.h>

#include <cmath>
#include <mutex>
#include <type_traits>

namespace koemi {

// The rocBLAS handle of a device (blas.hip); callers hold g_blas_mutex.
rocblas_handle blas_handle(int device);
extern std::mutex g_blas_mutex;

namespace {

constexpr int kSoftmaxWaves = 4;
constexpr int64_t kFusedMaxSlots = 1024;  // the softmax kernel holds a row in registers (16 slots per lane)
constexpr int kParts = 4;                 // width parts of the scores kernel (partial sums added by the softmax)
constexpr int kChunk = 64;                // width columns of one wave task of the scores kernel

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

// Slot tiles (32 slots each) of query tile y that can hold an eligible slot
// for some query of the tile: slot s is eligible for query t only if
// s < S + t (and s >= S + t - window with a sliding window), so the tiles
// x in [first_slot_tile, first_slot_tile + active_slot_tiles) are needed:
// 32 x < S + t_max and 32 x + 31 >= S + t_min - window.
__host__ __device__ inline int first_slot_tile(int y, int S, int window) {
    return window > 0 ? max(0, (S + 32 * y - window) / 32) : 0;
}
__host__ __device__ inline int active_slot_tiles(int y, int S, int L, int K, int window) {
    const int t_max = min(32 * y + 31, L - 1);
    return max(0, min((K + 31) / 32, (S + t_max + 31) / 32) - first_slot_tile(y, S, window));
}

// Partial scores of one (32 slots, 32 queries, batch, quarter of the width)
// tile: partial[part][b][t][s] = (sum over the part's width columns of
// key_s . query_t) / sqrt(D). Only the tiles active_slot_tiles() names are
// launched; tile groups (batch, part) are laid out contiguously per XCD (the
// dispatcher deals workgroups to the 8 XCDs in turn) so one XCD's L2 serves
// every re-read of a batch's queries and keys.
//
// The four waves take 64-column chunks of the part in turn. Lane l (row
// r = l % 32, half h = l / 32) loads, straight from memory, eight four-element
// groups of query row r and key row r at columns 64 c + 32 blk + 16 h + 4 i;
// component j of group (blk, i) feeds one v_mfma_f32_32x32x2f32 step. A
// lane's query and key values sit at the same column and the step's two
// K-entries (h = 0, 1) at two distinct columns, so the 32 steps of a chunk
// cover its 64 columns once: the column order inside the sum is permuted,
// the sum is the same. VEC: width % 4 == 0 (four-element loads).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void salient_scores_kernel(
    const T* __restrict__ ck, const T* __restrict__ k, const T* __restrict__ q, float* __restrict__ partial,
    int B, int S, int L, int64_t D, float inv_sqrt_d, int tiles, int total, int per_xcd, int window) {
    const int pid = static_cast<int>(blockIdx.x);
    const int logical = (pid & 7) * per_xcd + (pid >> 3);
    if (logical >= total) return;
    const int group = logical / tiles;
    int rem = logical - group * tiles, y = 0;
    const int K = S + L;
    for (;; ++y) {
        const int n = active_slot_tiles(y, S, L, K, window);
        if (rem < n) break;
        rem -= n;
    }
    const int b = group / kParts, part = group % kParts;
    const int s0 = (first_slot_tile(y, S, window) + rem) * 32, q0 = y * 32;
    const int lane = lane_id(), wave = static_cast<int>(threadIdx.x) / kWave;
    const int r = lane & 31, h = lane >> 5;
    const int64_t nch = (D + kChunk - 1) / kChunk, per_part = (nch + kParts - 1) / kParts;
    const int64_t c_end = min(nch, (part + 1) * per_part);
    const T* qrow = q + (static_cast<int64_t>(b) * L + min(q0 + r, L - 1)) * D;
    const int sl = min(s0 + r, K - 1);
    const T* krow = sl < S ? ck + (static_cast<int64_t>(b) * S + sl) * D : k + (static_cast<int64_t>(b) * L + (sl - S)) * D;

    float4 qa[8], kb[8];
    auto load_chunk = [&](int64_t c) {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int64_t d = c * kChunk + 32 * (g / 4) + 16 * h + 4 * (g % 4);
            if constexpr (VEC) {
                const bool in = d < D;
                const int64_t dc = in ? d : 0;
                qa[g] = load4_f32(qrow + dc);
                kb[g] = load4_f32(krow + dc);
                if (!in) qa[g] = kb[g] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            } else {
                float x[4], z[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool in = d + j < D;
                    const int64_t dc = in ? d + j : 0;
                    x[j] = load_f32(qrow + dc);
                    z[j] = load_f32(krow + dc);
                    if (!in) x[j] = z[j] = 0.0f;
                }
                qa[g] = make_float4(x[0], x[1], x[2], x[3]);
                kb[g] = make_float4(z[0], z[1], z[2], z[3]);
            }
        }
    };
    // Two accumulators keep two MFMA chains in flight.
    f32x16 acc0, acc1;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc0[v] = acc1[v] = 0.0f;
    for (int64_t c = part * per_part + wave; c < c_end; c += 4) {
        load_chunk(c);
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[g].x, kb[g].x, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[g].y, kb[g].y, acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[g].z, kb[g].z, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[g].w, kb[g].w, acc1, 0, 0, 0);
        }
    }
    const f32x16 acc = acc0 + acc1;
    // Sum the four waves' tiles: element v of lane l is query
    // 8 (v / 4) + 4 (l / 32) + v % 4, slot l % 32.
    __shared__ float red[4][16][kWave];
#pragma unroll
    for (int v = 0; v < 16; ++v) red[wave][v][lane] = acc[v];
    __syncthreads();
#pragma unroll
    for (int vv = 0; vv < 4; ++vv) {
        const int v = wave * 4 + vv;
        const float sum = red[0][v][lane] + red[1][v][lane] + red[2][v][lane] + red[3][v][lane];
        const int t = q0 + 8 * (v / 4) + 4 * h + v % 4;
        const int slot = s0 + r;
        if (t < L && slot < K)
            partial[((static_cast<int64_t>(part) * B + b) * L + t) * K + slot] = sum * inv_sqrt_d;
    }
}

// Masked softmax of one query row per wave (b, t): the four partial scores
// are added (fixed order), slot s is eligible when its valid or admission
// byte is set and s < S + t (and s >= S + t - window when window > 0, the
// local memory's sliding window); weights = exp(score - max) / sum over the
// eligible slots, zero elsewhere and in rows with none, written as fp32 rows
// of pitch Kp (K rounded up to 32; the padding is zero). NJ x 64 >= Kp.
template <int NJ>
__global__ __launch_bounds__(256) void salient_softmax_kernel(
    const float* __restrict__ partial, const uint8_t* __restrict__ carried_valid,
    const uint8_t* __restrict__ admission, float* __restrict__ weight, int B, int S, int L, int Kp, int window) {
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;  // b L + t
    if (row >= static_cast<int64_t>(B) * L) return;
    const int b = static_cast<int>(row / L), t = static_cast<int>(row % L);
    const int K = S + L, lim = S + t, low = window > 0 ? lim - window : 0;
    const int64_t part_stride = static_cast<int64_t>(B) * L * K;
    const float* x0 = partial + row * K;
    float x[NJ];
    bool ok[NJ];
    float m = -INFINITY;
    bool any = false;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int sl = 64 * j + lane;
        if (64 * j < K) {
            const int slc = min(sl, K - 1);
            const bool f = (slc < S ? carried_valid[static_cast<int64_t>(b) * S + slc]
                                    : admission[static_cast<int64_t>(b) * L + (slc - S)]) != 0;
            float v = x0[slc];
#pragma unroll
            for (int p = 1; p < kParts; ++p) v += x0[p * part_stride + slc];
            x[j] = v;
            ok[j] = sl < K && f && sl < lim && sl >= low;
        } else {
            x[j] = 0.0f;
            ok[j] = false;
        }
        if (ok[j]) {
            any = true;
            m = fmaxf(m, x[j]);
        }
    }
    m = wave_max_xor(m);
    any = __any(any);
    if (!any) m = 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        x[j] = ok[j] ? expf(x[j] - m) : 0.0f;
        sum += x[j];
    }
    sum = wave_sum_xor(sum);
    float* w = weight + row * Kp;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int sl = 64 * j + lane;
        if (64 * j < Kp && sl < Kp) w[sl] = sum > 0.0f ? x[j] / sum : x[j];
    }
}

// One-position window (a decode step): the query attends to the carried
// slots only (window entries before position 0: none), those that are valid
// and, with a sliding window, not older than `window` entries. One workgroup
// per (batch row, 1024 columns): each wave scores a quarter of the slots over
// the whole width (four-element loads, all of a slot's loads in flight before
// the wave reduction), wave 0 forms the softmax in LDS, then each thread sums
// its four columns over the slots, eight slots' loads at a time. Needs
// width % 4 == 0 and aligned rows; otherwise the window kernels run.
constexpr int kStepMaxSlots = 256;

template <typename T>
struct Vec4 {
    __device__ static void load(const T* p, float (&o)[4]) {
        typedef __attribute__((__vector_size__(4 * sizeof(T)))) T t4;
        const t4 v = *reinterpret_cast<const t4*>(p);
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = to_f32(v[c]);
    }
    __device__ static void store(T* p, const float (&o)[4]) {
        typedef __attribute__((__vector_size__(4 * sizeof(T)))) T t4;
        t4 v;
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = from_f32<T>(o[c]);
        *reinterpret_cast<t4*>(p) = v;
    }
};

// One memory of a one-position read; blockIdx.z picks one of two (the HERM
// block's local and salient reads of the same query in one launch).
template <typename T>
struct StepMemory {
    const T* ck;
    const T* cv;
    const uint8_t* cvalid;
    T* out;
    int S;
    int window;
};

__device__ __forceinline__ void load4_any(const float* p, float (&o)[4]) { Vec4<float>::load(p, o); }
__device__ __forceinline__ void load4_any(const bf16* p, float (&o)[4]) {
    const float4 x = load4(p);
    o[0] = x.x;
    o[1] = x.y;
    o[2] = x.z;
    o[3] = x.w;
}

// The ring of one memory after a one-position window (fp32 rings of S == the
// capacity slots, the position's entry in KT rows kstride elements apart):
// tail = the last S entries of [ring ; entry] (LocalKeyValueMemory.tail,
// memory.py:385-403), rows as stored; otherwise the salient_tail rule of
// memory.py:431-455 (flag = admission, invalid slots zeroed). An entry whose
// kvalid byte is 0 enters as zeros (network.py:337-340).
template <typename KT>
struct StepRing {
    const KT* k;
    const KT* v;
    int64_t kstride;
    const uint8_t* kvalid;
    const uint8_t* flag;
    float* ok;
    float* ov;
    uint8_t* ovalid;
    bool tail;
};

struct NoRing {};

// Batch row b, columns [1024 col_block, + 1024) of the read (the scores
// always run over the whole width).
template <typename T, typename Ring = NoRing>
__device__ void read_step_body(const T* __restrict__ ck, const T* __restrict__ cv, const uint8_t* __restrict__ cvalid,
                               const T* __restrict__ q, T* __restrict__ out, int S, int64_t D, float inv_sqrt_d,
                               int window, int64_t b, int col_block, const Ring& ring = Ring{});

// The ring after a one-position window (see StepRing): slots [s_begin, s_end)
// of batch row b, columns [col_begin, col_end) (the slot selection is made
// over the whole ring by every workgroup that calls this; valid bytes are
// written by the one with col_begin == 0). 256 threads, four columns each.
template <typename KT>
__device__ void ring_step_body(const float* __restrict__ ck, const float* __restrict__ cv,
                               const uint8_t* __restrict__ cvalid, int S, int64_t D, int64_t b, int s_begin,
                               int s_end, int64_t col_begin, int64_t col_end, const StepRing<KT>& ring) {
    __shared__ uint8_t fl[kStepMaxSlots + 1];
    __shared__ int16_t slot_src[kStepMaxSlots];
    __shared__ uint8_t slot_flag[kStepMaxSlots];
    const int tid = threadIdx.x;
    const int N = S + 1, C = S;
    for (int i = tid; i < N; i += 256) fl[i] = (i < S ? cvalid[b * S + i] : ring.flag[b]) != 0 ? 1 : 0;
    __syncthreads();
    if (ring.tail) {
        for (int s = tid; s < C; s += 256) {
            slot_src[s] = static_cast<int16_t>(s + 1);
            slot_flag[s] = fl[s + 1];
        }
    } else {
        int total = 0;
        for (int j = 0; j < N; ++j) total += fl[j];
        const int m = min(total, C);
        for (int i = tid; i < N; i += 256) {
            int va = 0;
            for (int j = i + 1; j < N; ++j) va += fl[j];
            const int ia = (N - 1 - i) - va;
            const bool keep = fl[i] ? va < m : ia < C - m;
            if (keep) {
                const int slot = C - 1 - (min(va, m) + min(ia, C - m));
                slot_src[slot] = static_cast<int16_t>(i);
                slot_flag[slot] = fl[i];
            }
        }
    }
    __syncthreads();
    if (col_begin == 0)
        for (int s = s_begin + tid; s < s_end; s += 256) ring.ovalid[b * C + s] = slot_flag[s];
    const bool entry_zero = ring.kvalid != nullptr && ring.kvalid[b] == 0;
    for (int64_t d = col_begin + tid * 4; d < col_end; d += 1024) {
        float ek[4], ev[4];
        load4_any(ring.k + b * ring.kstride + d, ek);
        load4_any(ring.v + b * ring.kstride + d, ev);
        // sixteen slots at a time: every load in flight before the stores
        constexpr int kGroup = 16;
        for (int s0 = s_begin; s0 < s_end; s0 += kGroup) {
            float kq[kGroup][4], vq[kGroup][4];
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                const int s = s0 + u;
                const int i = s < s_end ? slot_src[s] : S;
                if (i < S) {
                    Vec4<float>::load(ck + (b * S + i) * D + d, kq[u]);
                    Vec4<float>::load(cv + (b * S + i) * D + d, vq[u]);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        kq[u][c] = ek[c];
                        vq[u][c] = ev[c];
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                const int s = s0 + u;
                if (s >= s_end) break;
                const bool zero = (!ring.tail && !slot_flag[s]) || (slot_src[s] == S && entry_zero);
                if (zero) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) kq[u][c] = vq[u][c] = 0.0f;
                }
                Vec4<float>::store(ring.ok + (b * C + s) * D + d, kq[u]);
                Vec4<float>::store(ring.ov + (b * C + s) * D + d, vq[u]);
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void read_step_kernel(const T* __restrict__ ck, const T* __restrict__ cv,
                                                        const uint8_t* __restrict__ cvalid,
                                                        const T* __restrict__ q, T* __restrict__ out, int S,
                                                        int64_t D, float inv_sqrt_d, int window) {
    read_step_body<T>(ck, cv, cvalid, q, out, S, D, inv_sqrt_d, window, blockIdx.x, static_cast<int>(blockIdx.y));
}

template <typename T>
__global__ __launch_bounds__(256) void read_step_pair_kernel(StepMemory<T> m0, StepMemory<T> m1,
                                                             const T* __restrict__ q, int64_t D, float inv_sqrt_d) {
    const StepMemory<T>& m = blockIdx.z == 0 ? m0 : m1;
    read_step_body<T>(m.ck, m.cv, m.cvalid, q, m.out, m.S, D, inv_sqrt_d, m.window, blockIdx.x,
                      static_cast<int>(blockIdx.y));
}

// read_step_pair_kernel that also writes both rings after the position
// (z = 0 the local ring, z = 1 the salient ring).
template <typename KT>
__global__ __launch_bounds__(256) void read_step_rings_kernel(StepMemory<float> m0, StepMemory<float> m1,
                                                              StepRing<KT> r0, StepRing<KT> r1,
                                                              const float* __restrict__ q, int64_t D,
                                                              float inv_sqrt_d) {
    const int cb = static_cast<int>(blockIdx.y);
    if (blockIdx.z == 0)
        read_step_body<float>(m0.ck, m0.cv, m0.cvalid, q, m0.out, m0.S, D, inv_sqrt_d, m0.window, blockIdx.x, cb, r0);
    else read_step_body<float>(m1.ck, m1.cv, m1.cvalid, q, m1.out, m1.S, D, inv_sqrt_d, m1.window, blockIdx.x, cb, r1);
}

// A decode step's whole memory in one launch: the two reads with their ring
// updates (read_step_rings_kernel) and the associative memory's read and
// update (step::assoc_step_body). Batch row blockIdx.x; blockIdx.y < 2 R (R =
// 1024-column blocks of the reads): memory y / R, column block y % R; past
// those, associative column block y - 2 R (256 columns each). The parts read
// nothing the others write.
struct AssocStep {
    int64_t stride, value_off, fk_off, fq_off, decay_off, write_off;
    const float* surprise;
    const uint8_t* valid;
    const float* basis;
    const float* normalizer;
    float* out;
    float* next_basis;
    float* next_normalizer;
    int M;
};

constexpr int kRingSlotsPerBlock = 4;  // ring slots copied by one workgroup of the combined launch

template <typename KT, int MAXM, typename PT>
__global__ __launch_bounds__(256) void decode_memory_kernel(StepMemory<float> m0, StepMemory<float> m1,
                                                            StepRing<KT> r0, StepRing<KT> r1,
                                                            const float* __restrict__ q, int64_t D, float inv_sqrt_d,
                                                            const PT* __restrict__ proj, AssocStep as, int R, int G) {
    const int y = static_cast<int>(blockIdx.y);
    const int64_t b = blockIdx.x;
    if (y < 2 * R) {
        if (y < R) read_step_body<float>(m0.ck, m0.cv, m0.cvalid, q, m0.out, m0.S, D, inv_sqrt_d, m0.window, b, y);
        else read_step_body<float>(m1.ck, m1.cv, m1.cvalid, q, m1.out, m1.S, D, inv_sqrt_d, m1.window, b, y - R);
    } else if (y < 2 * R + 2 * G) {
        const int g = (y - 2 * R) % G, s0 = g * kRingSlotsPerBlock;
        const StepMemory<float>& m = y - 2 * R < G ? m0 : m1;
        if (s0 >= m.S) return;  // uniform: this memory has fewer slot groups
        const int s1 = min(m.S, s0 + kRingSlotsPerBlock);
        if (y - 2 * R < G) ring_step_body(m0.ck, m0.cv, m0.cvalid, m0.S, D, b, s0, s1, 0, D, r0);
        else ring_step_body(m1.ck, m1.cv, m1.cvalid, m1.S, D, b, s0, s1, 0, D, r1);
    } else {
        step::assoc_step_body<MAXM, PT>(proj, as.stride, as.value_off, as.fk_off, as.fq_off, as.decay_off,
                                        as.write_off, as.surprise, as.valid, as.basis, as.normalizer, as.out,
                                        as.next_basis, as.next_normalizer, D, as.M, b, y - 2 * R - 2 * G);
    }
}

template <typename T, typename Ring>
__device__ void read_step_body(const T* __restrict__ ck, const T* __restrict__ cv, const uint8_t* __restrict__ cvalid,
                               const T* __restrict__ q, T* __restrict__ out, int S, int64_t D, float inv_sqrt_d,
                               int window, int64_t b, int col_block, const Ring& ring) {
    __shared__ float w_sh[kStepMaxSlots];
    __shared__ float stat[1];
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int low = window > 0 ? S - window : 0;
    const T* qb = q + b * D;
    // wave w scores slots w, w + 4, w + 8, w + 12 of each round of 16, all
    // their loads of a 1024-wide stretch in flight together
    for (int s0 = wave; s0 < S; s0 += 16) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int64_t d = lane * 4;
        for (; d + 3 * 256 < D; d += 4 * 256) {
            float qv[4][4], kv[4][4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) Vec4<T>::load(qb + d + u * 256, qv[u]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int sl = min(s0 + 4 * j, S - 1);  // past S: a valid row, result unused
#pragma unroll
                for (int u = 0; u < 4; ++u) Vec4<T>::load(ck + (b * S + sl) * D + d + u * 256, kv[j][u]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[j] = fmaf(kv[j][u][c], qv[u][c], acc[j]);
        }
        for (; d < D; d += 256) {
            float qv[4];
            Vec4<T>::load(qb + d, qv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float kv[4];
                Vec4<T>::load(ck + (b * S + min(s0 + 4 * j, S - 1)) * D + d, kv);
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[j] = fmaf(kv[c], qv[c], acc[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float sum = wave_sum_xor(acc[j]);
            const int sl = s0 + 4 * j;
            if (lane == 0 && sl < S) w_sh[sl] = (cvalid[b * S + sl] != 0 && sl >= low) ? sum * inv_sqrt_d : -INFINITY;
        }
    }
    __syncthreads();
    if (wave == 0) {
        float m = -INFINITY;
        for (int sl = lane; sl < S; sl += kWave) m = fmaxf(m, w_sh[sl]);
        m = wave_max_xor(m);
        float sum = 0.0f;
        for (int sl = lane; sl < S; sl += kWave) {
            const float x = w_sh[sl];
            const float ex = x == -INFINITY ? 0.0f : expf(x - m);
            w_sh[sl] = ex;
            sum += ex;
        }
        sum = wave_sum_xor(sum);
        if (lane == 0) stat[0] = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = stat[0];
    const int64_t d = static_cast<int64_t>(col_block) * 1024 + tid * 4;
    if (d < D) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const T* vcol = cv + b * S * D + d;
        int sl = 0;
        for (; sl + 8 <= S; sl += 8) {
            float v[8][4];
#pragma unroll
            for (int u = 0; u < 8; ++u) Vec4<T>::load(vcol + (sl + u) * D, v[u]);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float wgt = w_sh[sl + u] * inv;
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[c] = fmaf(wgt, v[u][c], acc[c]);
            }
        }
        for (; sl < S; ++sl) {
            float v[4];
            Vec4<T>::load(vcol + sl * D, v);
            const float wgt = w_sh[sl] * inv;
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[c] = fmaf(wgt, v[c], acc[c]);
        }
        Vec4<T>::store(out + b * D + d, acc);
    }
    if constexpr (!std::is_same<Ring, NoRing>::value)
        ring_step_body(ck, cv, cvalid, S, D, b, 0, S, static_cast<int64_t>(col_block) * 1024,
                       min(D, static_cast<int64_t>(col_block) * 1024 + 1024), ring);
}

// out[b][t][d] = sum over slots s of weight[b][t][s] . [carried_values ; values][b][s][d]
// for queries [q0, q0 + 32) and columns [d0, d0 + 128): eight waves, two per
// 32-column slice, each taking half of the 32-slot blocks (the second half's
// sums are added through LDS), v_mfma_f32_32x32x2f32. Lane l (row r, half h)
// loads four four-element groups of weight row r at slots 32 blk + 16 h + 4 i
// and the 16 value rows 32 blk + 16 h + s at column d0 + 32 w + r; step
// s = 4 i + j pairs component j of group i with value row s, so each lane's
// weight and value refer to the same slot. Blocks past the last slot that is
// eligible for some query of the tile (S + t_max), and with a sliding window
// the blocks before its first one, are skipped (their weights are zero);
// value rows are requested two blocks ahead of use.
template <typename T>
__global__ __launch_bounds__(512) void salient_pv_kernel(
    const float* __restrict__ weight, const T* __restrict__ cv, const T* __restrict__ v, T* __restrict__ out,
    int B, int S, int L, int64_t D, int Kp, int window) {
    const int64_t d0 = static_cast<int64_t>(blockIdx.x) * 128;
    const int q0 = static_cast<int>(blockIdx.y) * 32, b = static_cast<int>(blockIdx.z);
    const int lane = lane_id(), wave = static_cast<int>(threadIdx.x) / kWave;
    const int slice = wave & 3, second = wave >> 2;
    const int r = lane & 31, h = lane >> 5;
    const int K = S + L;
    const int t_max = min(q0 + 31, L - 1);
    const int all_blocks = (min(K, S + t_max) + 31) / 32;
    const int lo = min(first_slot_tile(q0 / 32, S, window), all_blocks);
    const int first_end = lo + (all_blocks - lo + 1) / 2;
    const int blk0 = second ? first_end : lo, blocks = second ? all_blocks : first_end;
    const float* wrow = weight + (static_cast<int64_t>(b) * L + min(q0 + r, L - 1)) * Kp + 16 * h;
    const int64_t dw = d0 + slice * 32;
    const int64_t dcol = min(dw + r, D - 1);
    const T* cv_b = cv + static_cast<int64_t>(b) * S * D + dcol;  // + slot * D (carried slots)
    const T* v_b = v + static_cast<int64_t>(b) * L * D + dcol;    // + (slot - S) * D (window slots)
    struct Block {
        float4 w[4];
        float val[16];
    };
    auto load_block = [&](Block& dst, int blk) {
        if (blk >= blocks) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) dst.w[i] = *reinterpret_cast<const float4*>(wrow + 32 * blk + 4 * i);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int sl = min(32 * blk + 16 * h + s, K - 1);  // clamped rows carry zero weight
            dst.val[s] = load_f32(sl < S ? cv_b + static_cast<int64_t>(sl) * D : v_b + static_cast<int64_t>(sl - S) * D);
        }
    };
    f32x16 acc0, acc1;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.0f;
    auto multiply = [&](const Block& src) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(src.w[i].x, src.val[4 * i + 0], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(src.w[i].y, src.val[4 * i + 1], acc1, 0, 0, 0);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(src.w[i].z, src.val[4 * i + 2], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(src.w[i].w, src.val[4 * i + 3], acc1, 0, 0, 0);
        }
    };
    Block ba, bb, bc;
    load_block(ba, blk0);
    load_block(bb, blk0 + 1);
    for (int blk = blk0; blk < blocks; blk += 3) {
        load_block(bc, blk + 2);
        multiply(ba);
        if (blk + 1 >= blocks) break;
        load_block(ba, blk + 3);
        multiply(bb);
        if (blk + 2 >= blocks) break;
        load_block(bb, blk + 4);
        multiply(bc);
    }
    f32x16 acc = acc0 + acc1;
    __shared__ float red[4][16][kWave];
    if (second) {
#pragma unroll
        for (int i = 0; i < 16; ++i) red[slice][i][lane] = acc[i];
    }
    __syncthreads();
    if (second) return;
    // Element i of lane l: query 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = q0 + 8 * (i / 4) + 4 * h + i % 4;
        const int64_t d = dw + r;
        if (t < L && d < D) out[(static_cast<int64_t>(b) * L + t) * D + d] = from_f32<T>(acc[i] + red[slice][i][lane]);
    }
}

template <typename T>
__global__ __launch_bounds__(kWave * kSoftmaxWaves) void masked_softmax_kernel(
    const float* __restrict__ score, const uint8_t* __restrict__ carried_valid, const uint8_t* __restrict__ admission,
    T* __restrict__ weight, int64_t B, int64_t S, int64_t L, int64_t window) {
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kSoftmaxWaves + threadIdx.x / kWave;  // b * L + t
    if (row >= B * L) return;
    const int64_t b = row / L, t = row % L;
    const int64_t K = S + L;
    const float* x = score + row * K;
    T* w = weight + row * K;
    auto eligible = [&](int64_t s) -> bool {
        if (window > 0 && s < S + t - window) return false;
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
    if (S + L <= kFusedMaxSlots) {  // the partial scores, then weight rows of pitch Kp
        const size_t kp = static_cast<size_t>((S + L + 31) / 32 * 32);
        w.weight_off = align(kParts * scores * sizeof(float));
        w.out_off = w.total = w.weight_off + align(rows * kp * sizeof(float));
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

namespace {

// Fused window read (fp32): one workgroup per (batch row, 32 queries) does
// the whole masked read of its queries in one launch. The candidate slots of
// the block (salient: every slot before its last query's own entry; local:
// the `window` entries before each query's own, a band of at most window + 31
// slots) are compacted by their flags (carried valid bytes, then the window's
// admission or valid bytes) into an LDS list, so slots that no query can use
// cost nothing (a row with nothing eligible only writes zeros). Then:
//   scores: 32 queries x the listed slots on fp32 MFMA (v_mfma_f32_32x32x2f32),
//     operands loaded straight from memory in the MFMA layout (a lane's query
//     and key values at the same width column, the step's two K entries at two
//     columns 16 apart), the four waves taking 64-column chunks in turn and
//     leaving their partial sums in LDS;
//   softmax: the partials added in wave order and scaled by 1/sqrt(D), masked
//     per query (salient: carried slots and earlier window entries; local:
//     the window before the query's own entry), max, exp, sum, weights in LDS;
//   weighted sum: out = weights x values of the listed slots on fp32 MFMA, each
//     wave taking 32-column tiles in turn, eight slot steps' value loads
//     issued together.
// Needs width % 4 == 0, 16-byte aligned rows and at most kWinMaxSlots
// candidate slots per block; other shapes take the kernels above.
constexpr int kWinQ = 32;
constexpr int kWinMaxSlots = 152;   // salient blocks: LDS 4 x 32 x 153 fp32 partial scores (78 KiB)
constexpr int kWinLocalSlots = 64;  // local blocks: 4 x 32 x 65 (33 KiB)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// x = hi + mid + lo exactly (fp32 into three bf16 parts, each the nearest to
// what the parts before it leave; the residuals are exact in fp32), so the
// products of the parts with a bf16 operand are exact in fp32 and the sum of
// the three partial dot products is the fp32 dot product up to the order of
// the additions.
__device__ __forceinline__ void split3(const float (&x)[8], bf16x8& hi, bf16x8& mid, bf16x8& lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const __bf16 a = static_cast<__bf16>(x[i]);
        const float r1 = x[i] - static_cast<float>(a);
        const __bf16 b = static_cast<__bf16>(r1);
        const float r2 = r1 - static_cast<float>(b);
        hi[i] = a;
        mid[i] = b;
        lo[i] = static_cast<__bf16>(r2);
    }
}

// eight values from column col (a multiple of 8) of a row, zeros past D (a
// multiple of 8)
__device__ __forceinline__ void load8(const float* row, int64_t col, int64_t D, float (&x)[8]) {
    if (col < D) {
        const float4 a = *reinterpret_cast<const float4*>(row + col);
        const float4 b = *reinterpret_cast<const float4*>(row + col + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.0f;
    }
}
__device__ __forceinline__ void load8(const bf16* row, int64_t col, int64_t D, float (&x)[8]) {
    if (col < D) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + col);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = static_cast<float>(v[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.0f;
    }
}

__device__ inline f32x16 mfma_f32_32x32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// out rows are `ostride` elements apart (the reads can land in a column
// block of a wider matrix, e.g. the fusion input in bf16). The window's keys
// and values are rows `kstride` elements apart of type KT (fp32, or the bf16
// columns of the block's projection read in place, widened exactly).
template <bool LOCAL, int MAXS, typename OutT, typename KT>
__global__ __launch_bounds__(256, LOCAL ? 2 : 1) void window_read_kernel(
    const float* __restrict__ ck, const float* __restrict__ cv, const uint8_t* __restrict__ cvalid,
    const KT* __restrict__ k, const KT* __restrict__ v, int64_t kstride, const uint8_t* __restrict__ flags,
    const float* __restrict__ q, OutT* __restrict__ out, int64_t ostride, int S, int L, int64_t D, int window,
    float scale) {
    constexpr int NST = (MAXS + 31) / 32;  // slot tiles
    constexpr int NJ = (MAXS + kWave - 1) / kWave;
    __shared__ int list[MAXS];
    __shared__ int wave_cnt[4], wave_carried[4];
    __shared__ float sc[4][kWinQ][MAXS + 1];
    const int64_t row = blockIdx.x;
    const int t0 = static_cast<int>(blockIdx.y) * kWinQ;
    const int nq = min(kWinQ, L - t0);
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int r = lane & 31, h = lane >> 5;
    // candidate slots [c_lo, c_hi): before the last query's own entry S + t0 + nq - 1
    const int c_hi = S + t0 + nq - 1;
    const int c_lo = LOCAL ? max(0, S + t0 - window) : 0;
    const int c = c_lo + tid;
    bool f = false;
    if (c < c_hi) f = (c < S ? cvalid[row * S + c] : flags[row * L + (c - S)]) != 0;
    const uint64_t bal = __ballot(f);
    const int before = __popcll(bal & ((1ull << lane) - 1ull));
    const uint64_t bal_carried = __ballot(f && c < S);
    if (lane == 0) {
        wave_cnt[wave] = __popcll(bal);
        wave_carried[wave] = __popcll(bal_carried);
    }
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += wave_cnt[w];
    const int n = wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    // the list is ascending: its first nc slots are carried ones
    const int nc = wave_carried[0] + wave_carried[1] + wave_carried[2] + wave_carried[3];
    if (f) list[base + before] = c;
    __syncthreads();
    OutT* orow0 = out + (row * L + t0) * ostride;
    if (n == 0) {  // nothing eligible for any query of the block: zero rows
        const int64_t quads = D / 4;
        for (int64_t i = tid; i < nq * quads; i += 256) {
            const int64_t m = i / quads;
            store4(orow0 + m * ostride + 4 * (i - m * quads), 0.0f, 0.0f, 0.0f, 0.0f);
        }
        return;
    }
    const int nst = (n + 31) / 32;
    // Rows of listed slots: carried rows (fp32, D apart) or window rows (KT,
    // kstride apart). Loads of a group of listed slots [i_lo, i_hi] take one
    // path when the group is all carried or all window (uniform: nc splits
    // the list), a per-lane choice only in the group that straddles nc.
    auto carried_row = [&](const float* base_rows, int s) { return base_rows + (row * S + s) * D; };
    auto window_row = [&](const KT* base_rows, int s) { return base_rows + (row * L + (s - S)) * kstride; };
    auto group_kind = [&](int i_lo, int i_hi) { return i_lo >= nc ? 1 : (min(i_hi, n - 1) < nc ? 0 : 2); };
    // scores
    {
        const float* qrow = q + (row * L + t0 + min(r, nq - 1)) * D;
        f32x16 acc[NST];
#pragma unroll
        for (int st = 0; st < NST; ++st)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[st][e] = 0.0f;
        // 64-column chunks; k step j of a chunk is columns 16 j .. 16 j + 15, of
        // which lane (r, h) holds the eight from 8 h (rows = queries, columns =
        // slots). The local read runs on bf16 MFMA with the queries split in
        // three (split3: exact products), three products per k step for bf16
        // window rows (keys read in place), six for fp32 rows; the salient read
        // (mostly carried slots) on fp32 MFMA, one product per column.
        const int64_t chunks = (D + 63) / 64;
        for (int64_t ch = wave; ch < chunks; ch += 4) {
            if constexpr (LOCAL) {
                // the queries as three bf16 parts (their sum is the query exactly)
                bf16x8 qh[4], qm[4], ql[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float x[8];
                    load8(qrow, 64 * ch + 16 * j + 8 * h, D, x);
                    split3(x, qh[j], qm[j], ql[j]);
                }
#pragma unroll
                for (int st = 0; st < NST; ++st) {
                    if (st >= nst) break;
                    const int ks = list[min(st * 32 + r, n - 1)];
                    bool window_only = false;
                    if constexpr (!std::is_same<KT, float>::value) window_only = group_kind(st * 32, st * 32 + 31) == 1;
                    if (window_only) {
                        // bf16 keys: three products per k step
                        const KT* krow = window_row(k, ks);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int64_t col = 64 * ch + 16 * j + 8 * h;
                            bf16x8 kb = {};
                            if (col < D) kb = *reinterpret_cast<const bf16x8*>(krow + col);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qh[j], kb, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qm[j], kb, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ql[j], kb, acc[st], 0, 0, 0);
                        }
                    } else {
                        // fp32 keys (carried slots) split as well: six products
                        // per k step (the three dropped are below 2^-24 of the
                        // product; for bf16 keys the last three add exact zeros)
                        float kx[4][8];
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int64_t col = 64 * ch + 16 * j + 8 * h;
                            if (ks < S) load8(carried_row(ck, ks), col, D, kx[j]);
                            else load8(window_row(k, ks), col, D, kx[j]);
                        }
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            bf16x8 kh, km, kl;
                            split3(kx[j], kh, km, kl);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qh[j], kh, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qm[j], kh, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ql[j], kh, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qh[j], km, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qm[j], km, acc[st], 0, 0, 0);
                            acc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qh[j], kl, acc[st], 0, 0, 0);
                        }
                    }
                }
            } else {
                // the salient read (mostly carried slots): fp32 MFMA, one product per column
                float qx[4][8];
#pragma unroll
                for (int j = 0; j < 4; ++j) load8(qrow, 64 * ch + 16 * j + 8 * h, D, qx[j]);
#pragma unroll
                for (int st = 0; st < NST; ++st) {
                    if (st >= nst) break;
                    const int ks = list[min(st * 32 + r, n - 1)];
                    float kx[4][8];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int64_t col = 64 * ch + 16 * j + 8 * h;
                        if (ks < S) load8(carried_row(ck, ks), col, D, kx[j]);
                        else load8(window_row(k, ks), col, D, kx[j]);
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int m = 0; m < 8; ++m) acc[st] = mfma_f32_32x32x2(qx[j][m], kx[j][m], acc[st]);
                }
            }
        }
        // accumulator entry e of lane l: query 8 (e / 4) + 4 h + e % 4, slot st * 32 + l % 32
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            if (st >= nst) break;
            if (st * 32 + r < n) {
#pragma unroll
                for (int e = 0; e < 16; ++e) sc[wave][8 * (e / 4) + 4 * h + (e % 4)][st * 32 + r] = acc[st][e];
            }
        }
    }
    __syncthreads();

    // softmax: wave w takes queries 8 w .. 8 w + 7; weights overwrite sc[0]
    for (int qq = 0; qq < 8; ++qq) {
        const int m = wave * 8 + qq;
        const int t = t0 + m;
        float x[NJ];
        bool ok[NJ];
        float mx = -INFINITY;
        bool any = false;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int idx = j * kWave + lane;
            x[j] = 0.0f;
            ok[j] = false;
            if (idx < n) {
                const int sl = list[idx];
                x[j] = (((sc[0][m][idx] + sc[1][m][idx]) + sc[2][m][idx]) + sc[3][m][idx]) * scale;
                ok[j] = m < nq && sl < S + t && (!LOCAL || sl >= S + t - window);
            }
            if (ok[j]) {
                any = true;
                mx = fmaxf(mx, x[j]);
            }
        }
        mx = wave_max_xor(mx);
        any = __any(any);
        if (!any) mx = 0.0f;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            x[j] = ok[j] ? expf(x[j] - mx) : 0.0f;
            sum += x[j];
        }
        sum = wave_sum_xor(sum);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int idx = j * kWave + lane;
            if (idx < n) sc[0][m][idx] = sum > 0.0f ? x[j] / sum : x[j];
        }
    }
    __syncthreads();

    // weighted sum of the listed slots' values: a wave covers 128 columns per
    // pass as four 32-column MFMA tiles (rows = queries, K = slots), lane
    // (r, h) feeding column 4 r + c of tile c; per group of 16 listed slots a
    // lane loads the 16-byte pieces (columns 4 r .. 4 r + 3) of slots 8 h ..
    // 8 h + 7, one group ahead of its use. The local read runs on bf16 MFMA
    // with the weights split in three (split3): three products for bf16 window
    // rows, six for fp32 rows (split as well); the salient read on fp32 MFMA.
    const int64_t passes = (D + 127) / 128;
    for (int64_t pc = wave; pc < passes; pc += 4) {
        const int64_t col = pc * 128 + 4 * r;
        const bool cok = col < D;
        const int64_t colc = cok ? col : 0;
        f32x16 o[4];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[cc][e] = 0.0f;
        float4 bn[8];
        auto fetch = [&](int i0) {
            auto fetch_with = [&](auto load_slot) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int li = i0 + 8 * h + u;
                    bn[u] = li < n ? load_slot(list[li]) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            };
            if constexpr (std::is_same<KT, float>::value) {
                fetch_with([&](int sl) { return load4((sl < S ? carried_row(cv, sl) : window_row(v, sl)) + colc); });
            } else {
                const int kind = group_kind(i0, i0 + 15);
                if (kind == 0) fetch_with([&](int sl) { return load4(carried_row(cv, sl) + colc); });
                else if (kind == 1) fetch_with([&](int sl) { return load4(window_row(v, sl) + colc); });
                else
                    fetch_with([&](int sl) {
                        return sl < S ? load4(carried_row(cv, sl) + colc) : load4(window_row(v, sl) + colc);
                    });
            }
        };
        fetch(0);
        // groups of 16 listed slots up to the last listed one (past it the
        // weights are zero: those groups would add exact zeros)
        for (int i0 = 0; i0 < n; i0 += 16) {
            float4 bc[8];
            float wv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                bc[u] = bn[u];
                const int li = i0 + 8 * h + u;
                wv[u] = li < n ? sc[0][r][li] : 0.0f;
            }
            if (i0 + 16 < n) fetch(i0 + 16);
            if constexpr (LOCAL) {
                bool bf16_rows = false;
                if constexpr (!std::is_same<KT, float>::value) bf16_rows = group_kind(i0, i0 + 15) == 1;
                bf16x8 wh, wm, wl;
                split3(wv, wh, wm, wl);
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    float vv[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        vv[u] = cc == 0 ? bc[u].x : cc == 1 ? bc[u].y : cc == 2 ? bc[u].z : bc[u].w;
                    if (bf16_rows) {
                        bf16x8 vb;  // exact: the rows hold bf16 values
#pragma unroll
                        for (int u = 0; u < 8; ++u) vb[u] = static_cast<__bf16>(vv[u]);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wh, vb, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wm, vb, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wl, vb, o[cc], 0, 0, 0);
                    } else {
                        bf16x8 vh, vm, vl;
                        split3(vv, vh, vm, vl);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wh, vh, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wm, vh, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wl, vh, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wh, vm, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wm, vm, o[cc], 0, 0, 0);
                        o[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wh, vl, o[cc], 0, 0, 0);
                    }
                }
            } else {
                // fp32 rows: one fp32 MFMA step per slot pair (slot 8 h + u of lane h)
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    o[0] = mfma_f32_32x32x2(wv[u], bc[u].x, o[0]);
                    o[1] = mfma_f32_32x32x2(wv[u], bc[u].y, o[1]);
                    o[2] = mfma_f32_32x32x2(wv[u], bc[u].z, o[2]);
                    o[3] = mfma_f32_32x32x2(wv[u], bc[u].w, o[3]);
                }
            }
        }
        if (cok) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = 8 * (e / 4) + 4 * h + (e % 4);
                if (m < nq) store4(orow0 + m * ostride + col, o[0][e], o[1][e], o[2][e], o[3][e]);
            }
        }
    }
}

// Whether the fused read takes a block: at most MAXS candidate slots.
inline bool window_read_fits(int64_t carried, int64_t length, int64_t window, int64_t width) {
    if (width % 8 != 0) return false;  // the scores' eight-column loads
    if (window > 0) return carried <= kWinLocalSlots && window + kWinQ - 1 <= kWinLocalSlots;
    return carried <= kWinMaxSlots && carried + length - 1 <= kWinMaxSlots;
}

template <typename OutT, typename KT = float>
int launch_window_read(const float* ck, const float* cv, const uint8_t* cvalid, const KT* k, const KT* v,
                       const uint8_t* flags, const float* q, OutT* out, int64_t ostride, int64_t batch,
                       int64_t carried, int64_t length, int64_t width, int64_t window, hipStream_t stream,
                       int64_t kstride = 0) {
    const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
    const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((length + kWinQ - 1) / kWinQ));
    if (kstride == 0) kstride = width;
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, ck, cv, cvalid, k, v, kstride, flags, q, out, ostride,
                           static_cast<int>(carried), static_cast<int>(length), width, static_cast<int>(window),
                           inv_sqrt_d);
    };
    if (window > 0) launch(window_read_kernel<true, kWinLocalSlots, OutT, KT>);
    else launch(window_read_kernel<false, kWinMaxSlots, OutT, KT>);
    return check_launch(window > 0 ? "koemi_local_read" : "koemi_salient_read");
}

// The masked read shared by the salient read (window 0: no lower bound) and
// the local memory's sliding-window read (window > 0).
int memory_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid, const void* keys,
                const void* values, const uint8_t* admission, const void* queries, void* out, int64_t batch,
                int64_t carried, int64_t length, int64_t width, int64_t window, int dtype, void* workspace,
                size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || carried < 0 || length < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "salient read needs non-negative batch, carried and length and positive width");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "salient read does not support dtype %s", dtype_name(dtype));
    if (window < 0 || window > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "memory read window outside [0, 2^31)");
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
    const size_t step_es = dtype == KOEMI_F32 ? 4 : 2;
    auto step_aligned = [&](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % (4 * step_es) == 0; };
    if (length == 1 && carried <= kStepMaxSlots && batch <= 65535 && width % 4 == 0 && step_aligned(carried_keys) &&
        step_aligned(carried_values) && step_aligned(queries) && step_aligned(out)) {
        // one position: only carried slots can be eligible
        const hipStream_t s1 = as_stream(stream);
        const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
        const int Si = static_cast<int>(carried), win = static_cast<int>(window);
        auto step = [&](auto tag) {
            using T = decltype(tag);
            hipLaunchKernelGGL(read_step_kernel<T>,
                               dim3(static_cast<unsigned>(batch), static_cast<unsigned>((width + 1023) / 1024)),
                               dim3(256), 0, s1,
                               static_cast<const T*>(carried_keys), static_cast<const T*>(carried_values),
                               carried_valid, static_cast<const T*>(queries), static_cast<T*>(out), Si, width,
                               inv_sqrt_d, win);
        };
        if (dtype == KOEMI_F32) step(float{});
        else if (dtype == KOEMI_F16) step(f16{});
        else step(bf16{});
        return check_launch("koemi_salient_read(one position)");
    }
    auto aligned16 = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (dtype == KOEMI_F32 && width % 4 == 0 && window_read_fits(carried, length, window, width) && batch <= 0x7fffffffLL &&
        (length + kWinQ - 1) / kWinQ <= 65535 &&
        aligned16(carried_keys) && aligned16(carried_values) && aligned16(keys) && aligned16(values) &&
        aligned16(queries) && aligned16(out)) {
        return launch_window_read(static_cast<const float*>(carried_keys), static_cast<const float*>(carried_values),
                                  carried_valid, static_cast<const float*>(keys), static_cast<const float*>(values),
                                  admission, static_cast<const float*>(queries), static_cast<float*>(out), width, batch,
                                  carried, length, width, window, as_stream(stream));
    }
    char* base = static_cast<char*>(workspace);
    float* score = reinterpret_cast<float*>(base + ws.score_off);
    void* weight = base + ws.weight_off;
    const hipStream_t s = as_stream(stream);

    if (K <= kFusedMaxSlots) {
        if (batch > 65535 || batch * length > 0x7fffffffLL / kParts || (width + 127) / 128 > 0x7fffffffLL)
            return fail(KOEMI_ERR_UNSUPPORTED, "salient read grid too large");
        const int Bi = static_cast<int>(batch), Si = static_cast<int>(carried), Li = static_cast<int>(length);
        const int Ki = static_cast<int>(K), Kp = (Ki + 31) / 32 * 32;
        int tiles = 0;
        const int win = static_cast<int>(window);
        for (int y = 0; y < (Li + 31) / 32; ++y) tiles += active_slot_tiles(y, Si, Li, Ki, win);
        const int64_t total = static_cast<int64_t>(tiles) * Bi * kParts;
        if (total > 0x3fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "salient read grid too large");
        const int per_xcd = static_cast<int>((total + 7) / 8);
        const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
        float* weight32 = reinterpret_cast<float*>(base + ws.weight_off);
        const int64_t rows = batch * length;
        const size_t esize = dtype == KOEMI_F32 ? 4 : 2;
        const bool vec = width % 4 == 0 && reinterpret_cast<uintptr_t>(queries) % (4 * esize) == 0 &&
                         reinterpret_cast<uintptr_t>(keys) % (4 * esize) == 0 &&
                         (carried == 0 || reinterpret_cast<uintptr_t>(carried_keys) % (4 * esize) == 0);
        auto run = [&](auto tag) {
            using T = decltype(tag);
            if (total > 0) {
                auto scores_kernel = [&](auto kernel) {
                    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(8 * per_xcd)), dim3(256), 0, s,
                                       static_cast<const T*>(carried_keys), static_cast<const T*>(keys),
                                       static_cast<const T*>(queries), score, Bi, Si, Li, width, inv_sqrt_d, tiles,
                                       static_cast<int>(total), per_xcd, win);
                };
                if (vec) scores_kernel(salient_scores_kernel<T, true>);
                else scores_kernel(salient_scores_kernel<T, false>);
            }
            auto softmax = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0, s, score,
                                   carried_valid, admission, weight32, Bi, Si, Li, Kp, static_cast<int>(window));
            };
            if (Kp <= 64) softmax(salient_softmax_kernel<1>);
            else if (Kp <= 128) softmax(salient_softmax_kernel<2>);
            else if (Kp <= 256) softmax(salient_softmax_kernel<4>);
            else if (Kp <= 512) softmax(salient_softmax_kernel<8>);
            else softmax(salient_softmax_kernel<16>);
            hipLaunchKernelGGL(salient_pv_kernel<T>,
                               dim3(static_cast<unsigned>((width + 127) / 128), static_cast<unsigned>((Li + 31) / 32),
                                    static_cast<unsigned>(Bi)),
                               dim3(512), 0, s, weight32, static_cast<const T*>(carried_values),
                               static_cast<const T*>(values), static_cast<T*>(out), Bi, Si, Li, width, Kp, win);
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
                               static_cast<float*>(weight), batch, carried, length, window);
            break;
        case KOEMI_F16:
            hipLaunchKernelGGL(masked_softmax_kernel<f16>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<f16*>(weight), batch, carried, length, window);
            break;
        default:
            hipLaunchKernelGGL(masked_softmax_kernel<bf16>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<bf16*>(weight), batch, carried, length, window);
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

}  // namespace

extern "C" int koemi_salient_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                                  const void* keys, const void* values, const uint8_t* admission, const void* queries,
                                  void* out, int64_t batch, int64_t carried, int64_t length, int64_t width, int dtype,
                                  void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    return memory_read(carried_keys, carried_values, carried_valid, keys, values, admission, queries, out, batch,
                       carried, length, width, 0, dtype, workspace, workspace_bytes, stream);
}

extern "C" int koemi_local_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                                const void* keys, const void* values, const uint8_t* valid, const void* queries,
                                void* out, int64_t batch, int64_t carried, int64_t length, int64_t width,
                                int64_t window, int dtype, void* workspace, size_t workspace_bytes,
                                koemi_stream_t stream) {
    if (window < 1) return fail(KOEMI_ERR_INVALID, "local read needs a positive window");
    return memory_read(carried_keys, carried_values, carried_valid, keys, values, valid, queries, out, batch, carried,
                       length, width, window, dtype, workspace, workspace_bytes, stream);
}

extern "C" int koemi_memory_read_into(const float* carried_keys, const float* carried_values,
                                      const uint8_t* carried_valid, const void* keys, const void* values,
                                      int key_dtype, int64_t key_row_stride, const uint8_t* flags,
                                      const float* queries, void* out, int out_dtype, int64_t out_row_stride,
                                      int64_t batch, int64_t carried, int64_t length, int64_t width, int64_t window,
                                      koemi_stream_t stream) {
    if (batch < 0 || carried < 0 || length < 0 || width < 1 || window < 0)
        return fail(KOEMI_ERR_INVALID, "memory read needs non-negative batch, carried, length and window, positive width");
    if (out_dtype != KOEMI_F32 && out_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "memory read output must be float32 or bfloat16");
    if (out_row_stride < width || out_row_stride % 4 != 0)
        return fail(KOEMI_ERR_INVALID, "memory read output row stride must be a multiple of 4, at least the width");
    if (key_dtype != KOEMI_F32 && key_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "memory read keys and values must be float32 or bfloat16");
    if (key_row_stride == 0) key_row_stride = width;
    if (key_row_stride < width || key_row_stride % 4 != 0)
        return fail(KOEMI_ERR_INVALID, "memory read key row stride must be a multiple of 4, at least the width");
    if (batch == 0 || length == 0) return KOEMI_OK;
    auto aligned16 = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (width % 4 != 0 || !window_read_fits(carried, length, window, width) || batch > 0x7fffffffLL ||
        (length + kWinQ - 1) / kWinQ > 65535 || !aligned16(carried_keys) || !aligned16(carried_values) ||
        !aligned16(keys) || reinterpret_cast<uintptr_t>(values) % (key_dtype == KOEMI_F32 ? 16 : 8) != 0 ||
        (key_dtype == KOEMI_BF16 && key_row_stride % 8 != 0) || !aligned16(queries) ||
        reinterpret_cast<uintptr_t>(out) % 8 != 0)
        return fail(KOEMI_ERR_UNSUPPORTED, "memory read into a strided output: shape outside the fused read");
    if (!keys || !values || !flags || !queries || !out || (carried > 0 && (!carried_keys || !carried_values ||
                                                                          !carried_valid)))
        return fail(KOEMI_ERR_INVALID, "memory read received a null pointer");
    auto run = [&](auto out_tag, auto key_tag) {
        using OutT = decltype(out_tag);
        using KT = decltype(key_tag);
        return launch_window_read(carried_keys, carried_values, carried_valid, static_cast<const KT*>(keys),
                                  static_cast<const KT*>(values), flags, queries, static_cast<OutT*>(out),
                                  out_row_stride, batch, carried, length, width, window, as_stream(stream),
                                  key_row_stride);
    };
    if (out_dtype == KOEMI_BF16) return key_dtype == KOEMI_BF16 ? run(bf16{}, bf16{}) : run(bf16{}, float{});
    return key_dtype == KOEMI_BF16 ? run(float{}, bf16{}) : run(float{}, float{});
}

extern "C" int koemi_read_step_pair(const float* local_keys, const float* local_values, const uint8_t* local_valid,
                                    int64_t local_slots, int64_t window, const float* salient_keys,
                                    const float* salient_values, const uint8_t* salient_valid, int64_t salient_slots,
                                    const float* queries, float* local_out, float* salient_out, int64_t batch,
                                    int64_t width, koemi_stream_t stream) {
    if (batch < 0 || width < 1 || local_slots < 0 || salient_slots < 0 || window < 1)
        return fail(KOEMI_ERR_INVALID, "read step pair needs non-negative sizes, a positive width and window");
    if (local_slots > kStepMaxSlots || salient_slots > kStepMaxSlots || width % 4 != 0 || batch > 65535 ||
        window > 0x7fffffffLL)
        return fail(KOEMI_ERR_UNSUPPORTED, "read step pair needs at most %d slots, width %% 4 == 0 and batch <= 65535",
                    kStepMaxSlots);
    if (batch == 0) return KOEMI_OK;
    auto aligned = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (!queries || !local_out || !salient_out || (local_slots > 0 && (!local_keys || !local_values || !local_valid)) ||
        (salient_slots > 0 && (!salient_keys || !salient_values || !salient_valid)))
        return fail(KOEMI_ERR_INVALID, "read step pair received a null pointer");
    if (!aligned(local_keys) || !aligned(local_values) || !aligned(salient_keys) || !aligned(salient_values) ||
        !aligned(queries) || !aligned(local_out) || !aligned(salient_out))
        return fail(KOEMI_ERR_INVALID, "read step pair needs 16-byte aligned rows");
    const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
    const StepMemory<float> m0{local_keys, local_values, local_valid, local_out, static_cast<int>(local_slots),
                               static_cast<int>(window)};
    const StepMemory<float> m1{salient_keys, salient_values, salient_valid, salient_out,
                               static_cast<int>(salient_slots), 0};
    hipLaunchKernelGGL(read_step_pair_kernel<float>,
                       dim3(static_cast<unsigned>(batch), static_cast<unsigned>((width + 1023) / 1024), 2),
                       dim3(256), 0, as_stream(stream), m0, m1, queries, width, inv_sqrt_d);
    return check_launch("koemi_read_step_pair");
}

extern "C" int koemi_read_step_pair_rings(
    const float* local_keys, const float* local_values, const uint8_t* local_valid, int64_t local_slots,
    int64_t window, const float* salient_keys, const float* salient_values, const uint8_t* salient_valid,
    int64_t salient_slots, const float* queries, float* local_out, float* salient_out, const void* keys,
    const void* values, int key_dtype, int64_t key_row_stride, const uint8_t* valid, const uint8_t* admission,
    float* next_local_keys, float* next_local_values, uint8_t* next_local_valid, float* next_salient_keys,
    float* next_salient_values, uint8_t* next_salient_valid, int64_t batch, int64_t width, koemi_stream_t stream) {
    if (batch < 0 || width < 1 || local_slots < 1 || salient_slots < 1 || window < 1)
        return fail(KOEMI_ERR_INVALID, "read step rings need non-negative batch, positive width, window and slots");
    if (local_slots > kStepMaxSlots || salient_slots > kStepMaxSlots || width % 4 != 0 || batch > 65535 ||
        window > 0x7fffffffLL)
        return fail(KOEMI_ERR_UNSUPPORTED, "read step rings need at most %d slots, width %% 4 == 0, batch <= 65535",
                    kStepMaxSlots);
    if (key_dtype != KOEMI_F32 && key_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "read step rings take float32 or bfloat16 keys and values");
    if (key_row_stride == 0) key_row_stride = width;
    if (key_row_stride < width || key_row_stride % 4 != 0)
        return fail(KOEMI_ERR_INVALID, "read step rings: key row stride must be a multiple of 4, at least the width");
    if (batch == 0) return KOEMI_OK;
    if (!queries || !local_out || !salient_out || !local_keys || !local_values || !local_valid || !salient_keys ||
        !salient_values || !salient_valid || !keys || !values || !valid || !admission || !next_local_keys ||
        !next_local_values || !next_local_valid || !next_salient_keys || !next_salient_values || !next_salient_valid)
        return fail(KOEMI_ERR_INVALID, "read step rings received a null pointer");
    auto aligned = [](const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
    const size_t ka = key_dtype == KOEMI_F32 ? 16 : 8;
    if (!aligned(local_keys, 16) || !aligned(local_values, 16) || !aligned(salient_keys, 16) ||
        !aligned(salient_values, 16) || !aligned(queries, 16) || !aligned(local_out, 16) ||
        !aligned(salient_out, 16) || !aligned(next_local_keys, 16) || !aligned(next_local_values, 16) ||
        !aligned(next_salient_keys, 16) || !aligned(next_salient_values, 16) || !aligned(keys, ka) ||
        !aligned(values, ka))
        return fail(KOEMI_ERR_INVALID, "read step rings need aligned rows");
    const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
    const StepMemory<float> m0{local_keys, local_values, local_valid, local_out, static_cast<int>(local_slots),
                               static_cast<int>(window)};
    const StepMemory<float> m1{salient_keys, salient_values, salient_valid, salient_out,
                               static_cast<int>(salient_slots), 0};
    const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>((width + 1023) / 1024), 2);
    auto launch = [&](auto tag) {
        using KT = decltype(tag);
        const StepRing<KT> r0{static_cast<const KT*>(keys), static_cast<const KT*>(values), key_row_stride, valid,
                              valid, next_local_keys, next_local_values, next_local_valid, true};
        const StepRing<KT> r1{static_cast<const KT*>(keys), static_cast<const KT*>(values), key_row_stride, valid,
                              admission, next_salient_keys, next_salient_values, next_salient_valid, false};
        hipLaunchKernelGGL(read_step_rings_kernel<KT>, grid, dim3(256), 0, as_stream(stream), m0, m1, r0, r1,
                           queries, width, inv_sqrt_d);
    };
    if (key_dtype == KOEMI_BF16) launch(bf16{});
    else launch(float{});
    return check_launch("koemi_read_step_pair_rings");
}

extern "C" int koemi_decode_memory_step(
    const float* local_keys, const float* local_values, const uint8_t* local_valid, int64_t local_slots,
    int64_t window, const float* salient_keys, const float* salient_values, const uint8_t* salient_valid,
    int64_t salient_slots, const float* queries, float* local_out, float* salient_out, const void* projections,
    int projection_dtype, int64_t row_stride, int64_t key_offset, int64_t value_offset, const uint8_t* valid,
    const uint8_t* admission, float* next_local_keys, float* next_local_values, uint8_t* next_local_valid,
    float* next_salient_keys, float* next_salient_values, uint8_t* next_salient_valid,
    int64_t assoc_value_offset, int64_t feature_offset, int64_t query_feature_offset, int64_t decay_offset,
    int64_t write_offset, const float* surprise, const float* basis, const float* normalizer, float* assoc_read,
    float* next_basis, float* next_normalizer, int64_t features, int64_t batch, int64_t width,
    koemi_stream_t stream) {
    if (batch < 0 || width < 1 || local_slots < 1 || salient_slots < 1 || window < 1 || features < 1)
        return fail(KOEMI_ERR_INVALID, "decode memory step needs positive width, window, slots and features");
    if (local_slots > kStepMaxSlots || salient_slots > kStepMaxSlots || width % 4 != 0 || batch > 65535 ||
        window > 0x7fffffffLL || features > 32)
        return fail(KOEMI_ERR_UNSUPPORTED,
                    "decode memory step needs at most %d slots, width %% 4 == 0, batch <= 65535, features <= 32",
                    kStepMaxSlots);
    if (projection_dtype != KOEMI_F32 && projection_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "decode memory step takes a float32 or bfloat16 projection");
    const int64_t cols = row_stride;
    auto inside = [&](int64_t off, int64_t n) { return off >= 0 && off + n <= cols; };
    if (row_stride % 4 != 0 || !inside(key_offset, width) || !inside(value_offset, width) ||
        !inside(assoc_value_offset, width) || !inside(feature_offset, features) ||
        !inside(query_feature_offset, features) || !inside(decay_offset, 1) || !inside(write_offset, 1) ||
        key_offset % 4 != 0 || value_offset % 4 != 0)
        return fail(KOEMI_ERR_INVALID, "decode memory step: projection columns outside the rows or misaligned");
    if (batch == 0) return KOEMI_OK;
    const void* ptrs[] = {queries, local_out, salient_out, local_keys, local_values, local_valid, salient_keys,
                          salient_values, salient_valid, projections, valid, admission, next_local_keys,
                          next_local_values, next_local_valid, next_salient_keys, next_salient_values,
                          next_salient_valid, surprise, basis, normalizer, assoc_read, next_basis, next_normalizer};
    for (const void* p : ptrs)
        if (!p) return fail(KOEMI_ERR_INVALID, "decode memory step received a null pointer");
    auto aligned = [](const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
    const size_t es = projection_dtype == KOEMI_F32 ? 4 : 2;
    if (!aligned(local_keys, 16) || !aligned(local_values, 16) || !aligned(salient_keys, 16) ||
        !aligned(salient_values, 16) || !aligned(queries, 16) || !aligned(local_out, 16) ||
        !aligned(salient_out, 16) || !aligned(next_local_keys, 16) || !aligned(next_local_values, 16) ||
        !aligned(next_salient_keys, 16) || !aligned(next_salient_values, 16) || !aligned(projections, 4 * es))
        return fail(KOEMI_ERR_INVALID, "decode memory step needs aligned rows");
    const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(width));
    const StepMemory<float> m0{local_keys, local_values, local_valid, local_out, static_cast<int>(local_slots),
                               static_cast<int>(window)};
    const StepMemory<float> m1{salient_keys, salient_values, salient_valid, salient_out,
                               static_cast<int>(salient_slots), 0};
    const AssocStep as{row_stride, assoc_value_offset, feature_offset, query_feature_offset, decay_offset,
                       write_offset, surprise, valid, basis, normalizer, assoc_read, next_basis, next_normalizer,
                       static_cast<int>(features)};
    const int R = static_cast<int>((width + 1023) / 1024);
    const int G = static_cast<int>(((local_slots > salient_slots ? local_slots : salient_slots) +
                                    kRingSlotsPerBlock - 1) / kRingSlotsPerBlock);
    const int assoc_blocks = static_cast<int>((width + 255) / 256);
    const dim3 grid(static_cast<unsigned>(batch), static_cast<unsigned>(2 * R + 2 * G + assoc_blocks));
    auto launch = [&](auto tag) {
        using KT = decltype(tag);
        const KT* base = static_cast<const KT*>(projections);
        const StepRing<KT> r0{base + key_offset, base + value_offset, row_stride, valid, valid, next_local_keys,
                              next_local_values, next_local_valid, true};
        const StepRing<KT> r1{base + key_offset, base + value_offset, row_stride, valid, admission,
                              next_salient_keys, next_salient_values, next_salient_valid, false};
        if (features <= 16)
            hipLaunchKernelGGL((decode_memory_kernel<KT, 16, KT>), grid, dim3(256), 0, as_stream(stream), m0, m1, r0,
                               r1, queries, width, inv_sqrt_d, base, as, R, G);
        else
            hipLaunchKernelGGL((decode_memory_kernel<KT, 32, KT>), grid, dim3(256), 0, as_stream(stream), m0, m1, r0,
                               r1, queries, width, inv_sqrt_d, base, as, R, G);
    };
    if (projection_dtype == KOEMI_BF16) launch(bf16{});
    else launch(float{});
    return check_launch("koemi_decode_memory_step");
}
