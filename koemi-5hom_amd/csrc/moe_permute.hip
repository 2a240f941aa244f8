// Stable MoE permutation for gfx950: a counting sort of (token, slot) pairs by
// expert that reproduces the order of a stable argsort bit for bit.
//
// Reference: cuda_kernels/moe/moe_kernels.cu:68-145, 390-499 (pair keys, CUB
// 64-bit radix sort, histogram, scan, gathers) and the stable-argsort oracle of
// model/experts.py:171-216. With E experts the key needs only log2(E+1) bits,
// so instead of eight radix passes over 64-bit keys this runs:
//
//   1. count   : one wave per chunk of kChunk pairs builds its per-expert
//                histogram in LDS (counts are order-independent);
//   2. scan    : one workgroup turns the [chunks, E+1] counts into
//                segment_offsets and the first destination of every
//                (chunk, expert) — chunk order then pair order is stability
//                (the table is staged in LDS when it fits);
//   3. scatter : each chunk walks its pairs in order, 64 at a time; lanes with
//                the same key are grouped with ballots, ranked by popcount of
//                the lower lanes, and advance an LDS cursor per key. Writes
//                sorted_rows / sorted_experts / sorted_weights and the pair ->
//                position map;
//   4. gather  : one wave per token reads its context row once and writes it to
//                each of its k positions (zero rows for invalid pairs, which
//                all land past segment_offsets[E]).
//
// Every destination is computed, none is claimed by an atomic, so the output
// does not depend on scheduling.
#include "common.hpp"
#include "moe_hash.hpp"

namespace koemi {
namespace {

constexpr int kChunk = 128;          // pairs per count/scatter wave
constexpr int kMaxExperts = 4095;    // LDS holds E+1 cursors (scan: E+1 int64)
constexpr int kScanThreads = 1024;
constexpr int kScanPerLane = 8;      // chunks per lane per scan block

inline int64_t num_chunks(int64_t pairs) { return (pairs + kChunk - 1) / kChunk; }

// Workspace layout (byte offsets, 256-aligned).
struct PermuteWorkspace {
    size_t counts_off, dest_off, total;
};
inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
inline PermuteWorkspace permute_workspace(int64_t tokens, int64_t k, int64_t E) {
    const int64_t pairs = tokens * k;
    PermuteWorkspace w;
    w.counts_off = 0;
    w.dest_off = align256(static_cast<size_t>(num_chunks(pairs) > 0 ? num_chunks(pairs) : 1) * (E + 1) * sizeof(int32_t));
    w.total = w.dest_off + align256(static_cast<size_t>(pairs > 0 ? pairs : 1) * sizeof(int64_t));
    return w;
}

// Where a pair's expert comes from: an assignments array [tokens, k] (ReadSrc)
// or the content hash of the pair's token and previous token, computed in place
// (HashSrc: the hash route of experts.py:283-289, so the assignments are never
// stored). Either way pair p is (token p / k, slot p % k).
template <typename I>
struct ReadSrc {
    const I* a;
    __device__ int64_t operator()(int64_t p) const { return static_cast<int64_t>(a[p]); }
};
template <typename I>
struct HashSrc {
    const I* tok;
    const I* prev;
    int64_t k, E;
    __device__ int64_t operator()(int64_t p) const {
        const int64_t t = p / k;
        const uint64_t h = content_hash(static_cast<int64_t>(tok[t]), static_cast<int64_t>(prev[t]));
        return hash_slot_expert(h, p - t * k, E);
    }
};

// Pair key (moe_kernels.cu:68-91) of pair g + lane: the expert for a valid token
// whose slot holds an in-range expert not already used by an earlier slot of the
// same token, else the sentinel E; -1 for lanes past p1. Earlier slots of a
// token are read from the lanes that hold them (pairs are token-major), with a
// memory read only when a token straddles the start of the 64-pair group.
template <typename Src>
__device__ __forceinline__ int32_t group_key(const Src a, const uint8_t* __restrict__ valid,
                                             int64_t g, int64_t p1, int64_t k, int64_t E) {
    const int lane = lane_id();
    const int64_t p = g + lane;
    const bool active = p < p1;
    const int64_t pc = active ? p : p1 - 1;
    const int64_t e = a(pc);
    const int64_t t = pc / k;
    const int64_t s = pc - t * k;
    bool ok = active && valid[t] && e >= 0 && e < E;
    for (int64_t r = 1; r < k; ++r) {
        const int64_t above = __shfl_up(e, static_cast<unsigned>(r < kWave ? r : 0), kWave);
        if (r <= s) {
            const int64_t earlier = (r < kWave && lane >= r) ? above : a(pc - r);
            ok = ok && earlier != e;
        }
    }
    return active ? static_cast<int32_t>(ok ? e : E) : -1;
}

template <typename Src>
__global__ __launch_bounds__(kWave) void permute_count_kernel(const Src a, const uint8_t* __restrict__ valid,
                                                              int32_t* __restrict__ counts, int64_t pairs, int64_t k,
                                                              int64_t E) {
    extern __shared__ int32_t hist[];
    const int64_t chunk = blockIdx.x;
    for (int64_t e = threadIdx.x; e <= E; e += kWave) hist[e] = 0;
    __syncthreads();
    const int64_t p0 = chunk * kChunk;
    const int64_t p1 = min(pairs, p0 + kChunk);
    for (int64_t g = p0; g < p1; g += kWave) {
        const int32_t key = group_key(a, valid, g, p1, k, E);
        if (key >= 0) atomicAdd(&hist[key], 1);
    }
    __syncthreads();
    int32_t* row = counts + chunk * (E + 1);
    for (int64_t e = threadIdx.x; e <= E; e += kWave) row[e] = hist[e];
}

// counts[c][e] -> first destination of (chunk c, key e); offsets[e] = first
// position of key e, offsets[E] = number of valid pairs. Each wave owns keys;
// a key's chunk counts are scanned kScanPerLane per lane with a wave prefix.
__global__ __launch_bounds__(kScanThreads) void permute_scan_kernel(int32_t* __restrict__ counts,
                                                                    int64_t* __restrict__ offsets, int64_t chunks,
                                                                    int64_t E) {
    extern __shared__ int64_t key_total[];  // E+1 entries
    __shared__ int64_t wave_tot[kScanThreads / kWave];
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    constexpr int kWaves = kScanThreads / kWave;
    const int64_t n = E + 1;
    // Sweep 1: total per key.
    for (int64_t key = wave; key < n; key += kWaves) {
        int64_t sum = 0;
        for (int64_t c0 = 0; c0 < chunks; c0 += kWave * kScanPerLane) {
            int32_t v[kScanPerLane];
            const int64_t cl = c0 + static_cast<int64_t>(lane) * kScanPerLane;
#pragma unroll
            for (int j = 0; j < kScanPerLane; ++j) v[j] = counts[(cl + j < chunks ? cl + j : chunks - 1) * n + key];
#pragma unroll
            for (int j = 0; j < kScanPerLane; ++j) sum += (cl + j < chunks) ? v[j] : 0;
        }
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, kWave);
        if (lane == 0) key_total[key] = sum;
    }
    __syncthreads();
    // Exclusive scan over keys: each thread scans a contiguous span.
    const int64_t per = (n + kScanThreads - 1) / kScanThreads;
    const int64_t b0 = min(n, tid * per), b1 = min(n, b0 + per);
    int64_t s = 0;
    for (int64_t e = b0; e < b1; ++e) s += key_total[e];
    int64_t total;
    int64_t run = block_exclusive_scan<kScanThreads>(s, wave_tot, total);
    for (int64_t e = b0; e < b1; ++e) {
        const int64_t v = key_total[e];
        key_total[e] = run;
        run += v;
    }
    __syncthreads();
    for (int64_t e = tid; e < n; e += kScanThreads) offsets[e] = key_total[e];
    // Sweep 2: exclusive scan of each key's counts over the chunks, from the key's offset.
    for (int64_t key = wave; key < n; key += kWaves) {
        int64_t base = key_total[key];
        for (int64_t c0 = 0; c0 < chunks; c0 += kWave * kScanPerLane) {
            int32_t v[kScanPerLane];
            const int64_t cl = c0 + static_cast<int64_t>(lane) * kScanPerLane;
#pragma unroll
            for (int j = 0; j < kScanPerLane; ++j) {
                const int64_t c = cl + j;
                v[j] = counts[(c < chunks ? c : chunks - 1) * n + key];
            }
            int64_t local = 0;
#pragma unroll
            for (int j = 0; j < kScanPerLane; ++j) local += (cl + j < chunks) ? v[j] : 0;
            int64_t incl = local;
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) {
                const int64_t up = __shfl_up(incl, off, kWave);
                if (lane >= off) incl += up;
            }
            int64_t pos = base + incl - local;
#pragma unroll
            for (int j = 0; j < kScanPerLane; ++j) {
                const int64_t c = cl + j;
                if (c < chunks) {
                    counts[c * n + key] = static_cast<int32_t>(pos);
                    pos += v[j];
                }
            }
            base += __shfl(incl, kWave - 1, kWave);
        }
    }
}

// The same scan with the whole [chunks, E+1] count table staged in LDS (when it
// fits and E + 1 <= 64): one coalesced read; per key, each lane sums a run of
// consecutive chunks and one 32-bit wave scan gives every lane's prefix (kept
// in LDS); the key offsets are scanned; each lane then writes the first
// destinations of its chunks; one coalesced write.
constexpr int kScanLdsInts = 12288;  // 48 KiB of counts
constexpr int kScanLdsKeys = 64;

__global__ __launch_bounds__(kScanThreads) void permute_scan_lds_kernel(int32_t* __restrict__ counts,
                                                                        int64_t* __restrict__ offsets, int chunks,
                                                                        int E) {
    __shared__ int32_t table[kScanLdsInts];
    __shared__ int32_t lane_prefix[kScanLdsKeys][kWave];
    __shared__ int32_t key_total[kScanLdsKeys];
    __shared__ int32_t wave_tot[kScanThreads / kWave];
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    constexpr int kWaves = kScanThreads / kWave;
    const int n = E + 1;
    const int total_ints = chunks * n;
    constexpr int kPer = kScanLdsInts / kScanThreads;
    {
        int32_t v[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {  // all loads in flight together, clamped
            const int i = j * kScanThreads + tid;
            v[j] = counts[i < total_ints ? i : total_ints - 1];
        }
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int i = j * kScanThreads + tid;
            if (i < total_ints) table[i] = v[j];
        }
    }
    __syncthreads();
    // Lane l of a key's wave owns chunks [l * run, (l + 1) * run).
    const int run = (chunks + kWave - 1) / kWave;
    const int c0 = lane * run, c1 = min(chunks, c0 + run);
    for (int key = wave; key < n; key += kWaves) {
        int32_t local = 0;
        for (int c = c0; c < c1; ++c) local += table[c * n + key];
        int32_t incl = local;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int32_t up = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += up;
        }
        lane_prefix[key][lane] = incl - local;
        if (lane == kWave - 1) key_total[key] = incl;
    }
    __syncthreads();
    int32_t total;
    const int32_t excl = block_exclusive_scan<kScanThreads>(tid < n ? key_total[tid] : 0, wave_tot, total);
    if (tid < n) offsets[tid] = excl;
    __syncthreads();  // key_total is rewritten below
    if (tid < n) key_total[tid] = excl;
    __syncthreads();
    for (int key = wave; key < n; key += kWaves) {
        int32_t pos = key_total[key] + lane_prefix[key][lane];
        for (int c = c0; c < c1; ++c) {
            const int32_t v = table[c * n + key];
            table[c * n + key] = pos;
            pos += v;
        }
    }
    __syncthreads();
    for (int i = tid; i < total_ints; i += kScanThreads) counts[i] = table[i];
}

template <typename Src>
__global__ __launch_bounds__(kWave) void permute_scatter_kernel(
    const Src a, const uint8_t* __restrict__ valid, const float* __restrict__ pair_w,
    const int32_t* __restrict__ bases, int64_t* __restrict__ sorted_rows, int64_t* __restrict__ sorted_experts,
    float* __restrict__ sorted_w, int64_t* __restrict__ dest, int64_t pairs, int64_t k, int64_t E) {
    extern __shared__ int32_t cursor[];
    const int64_t chunk = blockIdx.x;
    const int lane = lane_id();
    for (int64_t e = lane; e <= E; e += kWave) cursor[e] = bases[chunk * (E + 1) + e];
    __syncthreads();
    const int64_t p0 = chunk * kChunk;
    const int64_t p1 = min(pairs, p0 + kChunk);
    for (int64_t g = p0; g < p1; g += kWave) {
        const int64_t p = g + lane;
        const int32_t key = group_key(a, valid, g, p1, k, E);
        const bool active = key >= 0;
        // Group the lanes by key: peers = lanes of this group with my key.
        uint64_t remaining = __ballot(active);
        uint64_t peers = 0;
        while (remaining) {
            const int leader = __ffsll(static_cast<unsigned long long>(remaining)) - 1;
            const int32_t lkey = __shfl(key, leader, kWave);
            const uint64_t same = __ballot(active && key == lkey);
            if (active && key == lkey) peers = same;
            remaining &= ~same;
        }
        const int rank = __popcll(peers & lanemask_lt());
        int64_t d = 0;
        if (active) d = static_cast<int64_t>(cursor[key]) + rank;
        __syncthreads();
        if (active && rank == 0) cursor[key] += __popcll(peers);
        __syncthreads();
        if (active) {
            sorted_rows[d] = p / k;
            sorted_experts[d] = key;
            if (sorted_w) sorted_w[d] = (key < E) ? pair_w[p] : 0.0f;
            dest[p] = d;
        }
    }
}

template <typename T, bool VEC, bool NTS = false>
__global__ __launch_bounds__(kWave * 4) void permute_gather_kernel(const T* __restrict__ ctx,
                                                                   const int64_t* __restrict__ dest,
                                                                   const int64_t* __restrict__ offsets_end,
                                                                   T* __restrict__ out, int64_t tokens, int64_t k,
                                                                   int64_t D) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (t >= tokens) return;
    const int lane = lane_id();
    const int64_t valid_pairs = *offsets_end;
    const T* src = ctx + t * D;
    if constexpr (VEC) {
        constexpr int N = 16 / sizeof(T);
        const int64_t nvec = D / N;
        for (int64_t v0 = 0; v0 < nvec; v0 += kWave * 4) {
            uint4 buf[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {  // unconditional loads at clamped indices
                const int64_t v = v0 + u * kWave + lane;
                buf[u] = reinterpret_cast<const uint4*>(src)[v < nvec ? v : nvec - 1];
            }
            for (int64_t s = 0; s < k; ++s) {
                const int64_t d = dest[t * k + s];
                uint4* dst = reinterpret_cast<uint4*>(out + d * D);
                const bool keep = d < valid_pairs;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int64_t v = v0 + u * kWave + lane;
                    if (v < nvec) {
                        const uint4 val = keep ? buf[u] : make_uint4(0, 0, 0, 0);
                        if constexpr (NTS) store16_nt(dst + v, val);
                        else dst[v] = val;
                    }
                }
            }
        }
    } else {
        for (int64_t s = 0; s < k; ++s) {
            const int64_t d = dest[t * k + s];
            const bool keep = d < valid_pairs;
            for (int64_t c = lane; c < D; c += kWave) out[d * D + c] = keep ? src[c] : static_cast<T>(0.0f);
        }
    }
}

// Index phase of a small permutation (a decode step's pairs) in one
// workgroup: wave w keys pairs [64 w, 64 w + 64), counts each key's lanes with
// ballots (rank = earlier lanes with the same key), the waves' counts meet in
// LDS, and every pair's destination is
//   offset[key] + (same-key pairs of earlier waves) + rank,
// the same stable order as the chunked kernels.
constexpr int kSmallPairs = 1024;
constexpr int kSmallKeys = 64;  // E + 1

template <typename Src>
__global__ __launch_bounds__(kSmallPairs) void permute_small_kernel(
    const Src a, const uint8_t* __restrict__ valid, const float* __restrict__ pair_w,
    int64_t* __restrict__ sorted_rows, int64_t* __restrict__ sorted_experts, int64_t* __restrict__ offsets,
    float* __restrict__ sorted_w, int64_t* __restrict__ dest, int64_t pairs, int64_t k, int64_t E) {
    __shared__ int32_t wcount[kSmallPairs / kWave][kSmallKeys];
    __shared__ int32_t key_off[kSmallKeys];
    const int tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const int nkeys = static_cast<int>(E) + 1;
    for (int i = tid; i < (kSmallPairs / kWave) * kSmallKeys; i += kSmallPairs) (&wcount[0][0])[i] = 0;
    __syncthreads();
    const int64_t g = static_cast<int64_t>(wave) * kWave;
    int32_t key = -1;
    uint64_t peers = 0;
    if (g < pairs) {  // wave-uniform
        key = group_key(a, valid, g, pairs, k, E);
        const bool active = key >= 0;
        uint64_t remaining = __ballot(active);
        while (remaining) {
            const int leader = __ffsll(static_cast<unsigned long long>(remaining)) - 1;
            const int32_t lkey = __shfl(key, leader, kWave);
            const uint64_t same = __ballot(active && key == lkey);
            if (active && key == lkey) peers = same;
            remaining &= ~same;
        }
        if (active && __popcll(peers & lanemask_lt()) == 0) wcount[wave][key] = __popcll(peers);
    }
    __syncthreads();
    if (wave == 0) {
        // per key: the count of the earlier waves (in place), then the keys' exclusive offsets
        int32_t total = 0;
        if (lane < nkeys) {
            for (int w = 0; w < kSmallPairs / kWave; ++w) {
                const int32_t c = wcount[w][lane];
                wcount[w][lane] = total;
                total += c;
            }
        }
        int32_t incl = total;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int32_t up = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += up;
        }
        if (lane < nkeys) {
            key_off[lane] = incl - total;
            offsets[lane] = incl - total;
        }
    }
    __syncthreads();
    if (key >= 0) {
        const int64_t p = g + lane;
        const int64_t d = static_cast<int64_t>(key_off[key]) + wcount[wave][key] + __popcll(peers & lanemask_lt());
        sorted_rows[d] = p / k;
        sorted_experts[d] = key;
        if (sorted_w) sorted_w[d] = (key < E) ? pair_w[p] : 0.0f;
        dest[p] = d;
    }
}

template <typename Src>
int run_index_phase(const Src a, const uint8_t* valid, const float* pair_w, int64_t* sorted_rows,
                    int64_t* sorted_experts, int64_t* offsets, float* sorted_w, int32_t* counts, int64_t* dest,
                    int64_t pairs, int64_t k, int64_t E, hipStream_t s) {
    if (pairs <= kSmallPairs && E + 1 <= kSmallKeys) {
        hipLaunchKernelGGL(permute_small_kernel<Src>, dim3(1), dim3(kSmallPairs), 0, s, a, valid, pair_w, sorted_rows,
                           sorted_experts, offsets, sorted_w, dest, pairs, k, E);
        return check_launch("koemi_moe_permute(small)");
    }
    const int64_t chunks = num_chunks(pairs);
    const size_t hist_bytes = static_cast<size_t>(E + 1) * sizeof(int32_t);
    hipLaunchKernelGGL(permute_count_kernel<Src>, dim3(static_cast<unsigned>(chunks)), dim3(kWave), hist_bytes, s, a,
                       valid, counts, pairs, k, E);
    int st = check_launch("koemi_moe_permute(count)");
    if (st != KOEMI_OK) return st;
    if (chunks * (E + 1) <= kScanLdsInts && E + 1 <= kScanLdsKeys)
        hipLaunchKernelGGL(permute_scan_lds_kernel, dim3(1), dim3(kScanThreads), 0, s, counts, offsets,
                           static_cast<int>(chunks), static_cast<int>(E));
    else
        hipLaunchKernelGGL(permute_scan_kernel, dim3(1), dim3(kScanThreads), static_cast<size_t>(E + 1) * sizeof(int64_t),
                           s, counts, offsets, chunks, E);
    st = check_launch("koemi_moe_permute(scan)");
    if (st != KOEMI_OK) return st;
    hipLaunchKernelGGL(permute_scatter_kernel<Src>, dim3(static_cast<unsigned>(chunks)), dim3(kWave), hist_bytes, s, a,
                       valid, pair_w, counts, sorted_rows, sorted_experts, sorted_w, dest, pairs, k, E);
    return check_launch("koemi_moe_permute(scatter)");
}

template <typename T>
int run_gather(const void* ctx, const int64_t* dest, const int64_t* offsets_end, void* out, int64_t tokens, int64_t k,
               int64_t D, hipStream_t s) {
    const bool vec = (D * static_cast<int64_t>(sizeof(T))) % 16 == 0 && reinterpret_cast<uintptr_t>(ctx) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const dim3 grid(grid_for(tokens, 4)), block(kWave * 4);
    // the sorted context is written once and is far larger than the caches
    if (vec && tokens * k * D * static_cast<int64_t>(sizeof(T)) > KOEMI_NT_STORE_BYTES)
        hipLaunchKernelGGL((permute_gather_kernel<T, true, true>), grid, block, 0, s, static_cast<const T*>(ctx), dest,
                           offsets_end, static_cast<T*>(out), tokens, k, D);
    else if (vec)
        hipLaunchKernelGGL((permute_gather_kernel<T, true>), grid, block, 0, s, static_cast<const T*>(ctx), dest,
                           offsets_end, static_cast<T*>(out), tokens, k, D);
    else
        hipLaunchKernelGGL((permute_gather_kernel<T, false>), grid, block, 0, s, static_cast<const T*>(ctx), dest,
                           offsets_end, static_cast<T*>(out), tokens, k, D);
    return check_launch("koemi_moe_permute(gather)");
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" size_t koemi_moe_permute_workspace_bytes(int64_t tokens, int64_t top_k, int64_t expert_count) {
    if (tokens < 0 || top_k < 1 || expert_count < 1) return 0;
    return permute_workspace(tokens, top_k, expert_count).total;
}

extern "C" int koemi_moe_permute(const void* context, int context_dtype, const void* assignments,
                                 int assignment_dtype, const uint8_t* valid_mask, const float* pair_weights,
                                 void* sorted_context, int64_t* sorted_rows, int64_t* sorted_experts,
                                 int64_t* segment_offsets, float* sorted_weights, int64_t tokens, int64_t width,
                                 int64_t top_k, int64_t expert_count, void* workspace, size_t workspace_bytes,
                                 koemi_stream_t stream) {
    if (tokens < 1 || width < 1) return fail(KOEMI_ERR_INVALID, "context dimensions must be positive");
    if (top_k < 1 || top_k > 256) return fail(KOEMI_ERR_INVALID, "assignments top_k is outside [1, 256]");
    if (expert_count < 1 || top_k > expert_count) return fail(KOEMI_ERR_INVALID, "top_k must not exceed expert_count");
    if (expert_count > kMaxExperts) return fail(KOEMI_ERR_UNSUPPORTED, "permute supports at most %d experts", kMaxExperts);
    if (!float_dtype(context_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "context must be float32, float16 or bfloat16");
    if (!index_dtype(assignment_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "assignments must be int32 or int64");
    if ((pair_weights == nullptr) != (sorted_weights == nullptr))
        return fail(KOEMI_ERR_INVALID, "pair_weights and sorted_weights must both be given or both be null");
    if (!context || !assignments || !valid_mask || !sorted_rows || !sorted_experts || !segment_offsets)
        return fail(KOEMI_ERR_INVALID, "permute received a null pointer");
    const PermuteWorkspace ws = permute_workspace(tokens, top_k, expert_count);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "permute workspace too small: need %zu bytes", ws.total);
    if (num_chunks(tokens * top_k) > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many pairs");
    char* base = static_cast<char*>(workspace);
    int32_t* counts = reinterpret_cast<int32_t*>(base + ws.counts_off);
    int64_t* dest = reinterpret_cast<int64_t*>(base + ws.dest_off);
    hipStream_t s = as_stream(stream);
    const int64_t pairs = tokens * top_k;
    int st = (assignment_dtype == KOEMI_I32)
                 ? run_index_phase(ReadSrc<int32_t>{static_cast<const int32_t*>(assignments)}, valid_mask, pair_weights, sorted_rows, sorted_experts,
                                            segment_offsets, sorted_weights, counts, dest, pairs, top_k, expert_count, s)
                 : run_index_phase(ReadSrc<int64_t>{static_cast<const int64_t*>(assignments)}, valid_mask, pair_weights, sorted_rows, sorted_experts,
                                            segment_offsets, sorted_weights, counts, dest, pairs, top_k, expert_count, s);
    if (st != KOEMI_OK) return st;
    if (sorted_context == nullptr) return KOEMI_OK;  // the indices only (the caller reads rows by sorted_rows)
    const int64_t* offsets_end = segment_offsets + expert_count;
    switch (context_dtype) {
        case KOEMI_F32: return run_gather<float>(context, dest, offsets_end, sorted_context, tokens, top_k, width, s);
        case KOEMI_F16: return run_gather<f16>(context, dest, offsets_end, sorted_context, tokens, top_k, width, s);
        default: return run_gather<bf16>(context, dest, offsets_end, sorted_context, tokens, top_k, width, s);
    }
}

extern "C" int koemi_moe_permute_indices(const void* assignments, int assignment_dtype, const uint8_t* valid_mask,
                                         const float* pair_weights, int64_t* sorted_rows, int64_t* sorted_experts,
                                         int64_t* segment_offsets, float* sorted_weights, int64_t* pair_positions,
                                         int64_t tokens, int64_t top_k, int64_t expert_count, void* workspace,
                                         size_t workspace_bytes, koemi_stream_t stream) {
    if (tokens < 1) return fail(KOEMI_ERR_INVALID, "permute needs tokens >= 1");
    if (top_k < 1 || top_k > 256) return fail(KOEMI_ERR_INVALID, "assignments top_k is outside [1, 256]");
    if (expert_count < 1 || top_k > expert_count) return fail(KOEMI_ERR_INVALID, "top_k must not exceed expert_count");
    if (expert_count > kMaxExperts) return fail(KOEMI_ERR_UNSUPPORTED, "permute supports at most %d experts", kMaxExperts);
    if (!index_dtype(assignment_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "assignments must be int32 or int64");
    if ((pair_weights == nullptr) != (sorted_weights == nullptr))
        return fail(KOEMI_ERR_INVALID, "pair_weights and sorted_weights must both be given or both be null");
    if (!assignments || !valid_mask || !sorted_rows || !sorted_experts || !segment_offsets || !pair_positions)
        return fail(KOEMI_ERR_INVALID, "permute received a null pointer");
    const PermuteWorkspace ws = permute_workspace(tokens, top_k, expert_count);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "permute workspace too small: need %zu bytes", ws.total);
    if (num_chunks(tokens * top_k) > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many pairs");
    int32_t* counts = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + ws.counts_off);
    hipStream_t s = as_stream(stream);
    const int64_t pairs = tokens * top_k;
    return (assignment_dtype == KOEMI_I32)
               ? run_index_phase(ReadSrc<int32_t>{static_cast<const int32_t*>(assignments)}, valid_mask, pair_weights, sorted_rows, sorted_experts,
                                          segment_offsets, sorted_weights, counts, pair_positions, pairs, top_k,
                                          expert_count, s)
               : run_index_phase(ReadSrc<int64_t>{static_cast<const int64_t*>(assignments)}, valid_mask, pair_weights, sorted_rows, sorted_experts,
                                          segment_offsets, sorted_weights, counts, pair_positions, pairs, top_k,
                                          expert_count, s);
}

extern "C" int koemi_moe_permute_hash_indices(const void* token_ids, const void* previous_token_ids, int id_dtype,
                                              const uint8_t* valid_mask, int64_t* sorted_rows,
                                              int64_t* sorted_experts, int64_t* segment_offsets,
                                              int64_t* pair_positions, int64_t tokens, int64_t top_k,
                                              int64_t expert_count, void* workspace, size_t workspace_bytes,
                                              koemi_stream_t stream) {
    if (tokens < 1) return fail(KOEMI_ERR_INVALID, "permute needs tokens >= 1");
    if (top_k < 1 || top_k > 256) return fail(KOEMI_ERR_INVALID, "top_k is outside [1, 256]");
    if (expert_count < 1 || top_k > expert_count) return fail(KOEMI_ERR_INVALID, "top_k must not exceed expert_count");
    if (expert_count > kMaxExperts) return fail(KOEMI_ERR_UNSUPPORTED, "permute supports at most %d experts", kMaxExperts);
    if (!index_dtype(id_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "token ids must be int32 or int64");
    if (!token_ids || !previous_token_ids || !valid_mask || !sorted_rows || !sorted_experts || !segment_offsets ||
        !pair_positions)
        return fail(KOEMI_ERR_INVALID, "permute received a null pointer");
    const PermuteWorkspace ws = permute_workspace(tokens, top_k, expert_count);
    if (!workspace || workspace_bytes < ws.total)
        return fail(KOEMI_ERR_INVALID, "permute workspace too small: need %zu bytes", ws.total);
    if (num_chunks(tokens * top_k) > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "too many pairs");
    int32_t* counts = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + ws.counts_off);
    hipStream_t s = as_stream(stream);
    const int64_t pairs = tokens * top_k;
    if (id_dtype == KOEMI_I32)
        return run_index_phase(HashSrc<int32_t>{static_cast<const int32_t*>(token_ids),
                                                static_cast<const int32_t*>(previous_token_ids), top_k, expert_count},
                               valid_mask, nullptr, sorted_rows, sorted_experts, segment_offsets, nullptr, counts,
                               pair_positions, pairs, top_k, expert_count, s);
    return run_index_phase(HashSrc<int64_t>{static_cast<const int64_t*>(token_ids),
                                            static_cast<const int64_t*>(previous_token_ids), top_k, expert_count},
                           valid_mask, nullptr, sorted_rows, sorted_experts, segment_offsets, nullptr, counts,
                           pair_positions, pairs, top_k, expert_count, s);
}
