// MoE routing for gfx950: content-hash top-k, learned softmax top-k, device-side
// contract checks and per-expert activation counts.
//
// Reference: model/experts.py:30-38, 283-289 (hash route in int64),
// cuda_kernels/moe/moe_kernels.cu:33-66 (native route), model/router.py:43-59
// (learned gate), cuda_kernels/moe/__init__.py:113-125, 213-220 (checks) and
// model/network.py:48-70 (activation counts). All of it is integer work or a
// 16-wide softmax per token: one thread per token, no HBM-heavy traffic.
#include "common.hpp"
#include "detmath.hpp"
#include "moe_hash.hpp"

namespace koemi {
namespace {

template <typename I>
__global__ void route_hash_kernel(const I* __restrict__ tok, const I* __restrict__ prev,
                                  const uint8_t* __restrict__ valid, int64_t* __restrict__ out,
                                  int32_t* __restrict__ dup_flag, int64_t T, int64_t E, int64_t k) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    int64_t* row = out + t * k;
    if (!valid[t]) {
        for (int64_t s = 0; s < k; ++s) row[s] = -1;
        return;
    }
    const uint64_t h = content_hash(static_cast<int64_t>(tok[t]), static_cast<int64_t>(prev[t]));
    bool dup = false;
    for (int64_t s = 0; s < k; ++s) {
        const int64_t e = hash_slot_expert(h, s, E);
        for (int64_t r = 0; r < s; ++r) dup |= (row[r] == e);
        row[s] = e;
    }
    if (dup && dup_flag != nullptr) atomicOr(dup_flag, 1);
}

// The synthetic "token id mod E" route of the benchmark's hash variant: slot s
// of a valid token takes expert (tok + s) mod E, with torch.remainder's sign
// (the result is in [0, E) for negative ids too); invalid tokens -1. There is
// no counterpart in the reference (its hash route is route_hash_kernel above).
template <typename I>
__global__ void route_modulo_kernel(const I* __restrict__ tok, const uint8_t* __restrict__ valid,
                                    int64_t* __restrict__ out, int64_t T, int64_t E, int64_t k) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    int64_t* row = out + t * k;
    const int64_t base = valid[t] ? static_cast<int64_t>(tok[t]) % E : 0;
    for (int64_t s = 0; s < k; ++s) {
        int64_t e = (base + s) % E;
        e += e < 0 ? E : 0;
        row[s] = valid[t] ? e : -1;
    }
}

// softmax(logits) then top-k in descending probability, ties to the lower index
// (router.py:46-49). Probabilities use the fixed exp of detmath.hpp and a
// left-to-right sum so that weights are reproducible bit for bit.
//
// softmax_terms: the row max and the left-to-right sum of exp(l - max) of one
// token's logits.
__device__ __forceinline__ void softmax_terms(const float* __restrict__ l, int64_t E, float& m, float& sum) {
#pragma clang fp contract(off)
    m = -__builtin_inff();
    for (int64_t j = 0; j < E; ++j) m = fmaxf(m, l[j]);
    sum = 0.0f;
    for (int64_t j = 0; j < E; ++j) sum = sum + detmath::det_expf_nonpos(l[j] - m);
}

// The k largest probabilities of one valid token in descending order, ties to
// the lower expert index; returns nothing, writes idx[0..k) and wt[0..k).
__device__ __forceinline__ void learned_topk(const float* __restrict__ l, int64_t E, int64_t k, float m, float sum,
                                             int64_t* __restrict__ idx, float* __restrict__ wt) {
#pragma clang fp contract(off)
    float prev_p = __builtin_inff();
    int64_t prev_j = -1;
    for (int64_t s = 0; s < k; ++s) {
        int64_t best = -1;
        float best_p = 0.0f;
        for (int64_t j = 0; j < E; ++j) {
            const float p = detmath::det_expf_nonpos(l[j] - m) / sum;
            const bool after_prev = (p < prev_p) || (p == prev_p && j > prev_j);
            if (after_prev && (best < 0 || p > best_p)) {
                best = j;
                best_p = p;
            }
        }
        idx[s] = best;
        wt[s] = best < 0 ? 0.0f : best_p;
        prev_p = best_p;
        prev_j = best;
    }
}

__global__ void route_learned_kernel(const float* __restrict__ logits, const uint8_t* __restrict__ valid,
                                     int64_t* __restrict__ out_idx, float* __restrict__ out_w, int64_t T,
                                     int64_t E, int64_t k) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    int64_t* idx = out_idx + t * k;
    float* wt = out_w + t * k;
    if (!valid[t]) {
        for (int64_t s = 0; s < k; ++s) {
            idx[s] = -1;
            wt[s] = 0.0f;
        }
        return;
    }
    const float* l = logits + t * E;
    float m, sum;
    softmax_terms(l, E, m, sum);
    learned_topk(l, E, k, m, sum, idx, wt);
}

// The learned route with the RouterStatistics of router.py:11-22, 50-58 per
// workgroup of 256 tokens (one per thread, the same bits as
// route_learned_kernel): the probability mass of every expert over the
// workgroup's valid tokens, summed in token order (the probabilities staged in
// LDS by chunks of 64 experts, one thread per expert summing its column), the
// number of valid assignments per expert (integer LDS atomics: exact) and the
// number of valid tokens. router_stats_finish_kernel adds the workgroups'
// partials in workgroup order, so every result is a fixed function of the
// inputs.
constexpr int kStatThreads = 256;
constexpr int kStatChunk = 64;
constexpr int kStatMaxExperts = 1024;

__global__ __launch_bounds__(kStatThreads) void route_learned_stats_kernel(
    const float* __restrict__ logits, const uint8_t* __restrict__ valid, int64_t* __restrict__ out_idx,
    float* __restrict__ out_w, int64_t T, int64_t E, int64_t k, float* __restrict__ part_mass,
    uint32_t* __restrict__ part_counts, uint32_t* __restrict__ part_valid) {
#pragma clang fp contract(off)
    __shared__ float p_sh[kStatChunk][kStatThreads + 1];
    __shared__ uint32_t count_sh[kStatMaxExperts];
    __shared__ uint32_t valid_sh;
    const int tid = threadIdx.x;
    const int64_t blk = blockIdx.x;
    const int64_t t = blk * kStatThreads + tid;
    for (int64_t e = tid; e < E; e += kStatThreads) count_sh[e] = 0u;
    if (tid == 0) valid_sh = 0u;
    __syncthreads();
    const bool ok = t < T && valid[t];
    const float* l = logits + (ok ? t : 0) * E;
    float m = 0.0f, sum = 1.0f;
    if (t < T) {
        int64_t* idx = out_idx + t * k;
        float* wt = out_w + t * k;
        if (ok) {
            softmax_terms(l, E, m, sum);
            learned_topk(l, E, k, m, sum, idx, wt);
            for (int64_t s = 0; s < k; ++s)  // (no expert is picked only for NaN probabilities)
                if (idx[s] >= 0) atomicAdd(&count_sh[idx[s]], 1u);
            atomicAdd(&valid_sh, 1u);
        } else {
            for (int64_t s = 0; s < k; ++s) {
                idx[s] = -1;
                wt[s] = 0.0f;
            }
        }
    }
    for (int64_t c0 = 0; c0 < E; c0 += kStatChunk) {
        const int64_t n = E - c0 < kStatChunk ? E - c0 : kStatChunk;
        for (int64_t j = 0; j < n; ++j)
            p_sh[j][tid] = ok ? detmath::det_expf_nonpos(l[c0 + j] - m) / sum : 0.0f;
        __syncthreads();
        if (tid < n) {
            float acc = 0.0f;
            for (int i = 0; i < kStatThreads; ++i) acc = acc + p_sh[tid][i];
            part_mass[blk * E + c0 + tid] = acc;
        }
        __syncthreads();
    }
    for (int64_t e = tid; e < E; e += kStatThreads) part_counts[blk * E + e] = count_sh[e];
    if (tid == 0) part_valid[blk] = valid_sh;
}

// RouterStatistics.balance_loss (router.py:17-22) in fp32, in expert order:
// E * sum_e (mass_e / max(valid, 1)) * (counts_e / max(sum counts, 1)).
__device__ float balance_loss_of(const float* __restrict__ mass, const float* __restrict__ counts, float valid_count,
                                 int64_t E) {
#pragma clang fp contract(off)
    const float count = fmaxf(valid_count, 1.0f);
    float total = 0.0f;
    for (int64_t e = 0; e < E; ++e) total = total + counts[e];
    const float denom = fmaxf(total, 1.0f);
    float acc = 0.0f;
    for (int64_t e = 0; e < E; ++e) acc = acc + (mass[e] / count) * (counts[e] / denom);
    return static_cast<float>(E) * acc;
}

__global__ __launch_bounds__(kStatThreads) void router_stats_finish_kernel(
    const float* __restrict__ part_mass, const uint32_t* __restrict__ part_counts,
    const uint32_t* __restrict__ part_valid, int64_t blocks, int64_t E, float* __restrict__ mass,
    float* __restrict__ counts, float* __restrict__ valid_count, float* __restrict__ loss) {
#pragma clang fp contract(off)
    __shared__ float mass_sh[kStatMaxExperts];
    __shared__ float counts_sh[kStatMaxExperts];
    __shared__ float valid_sh;
    const int tid = threadIdx.x;
    for (int64_t e = tid; e < E; e += kStatThreads) {
        float acc = 0.0f;
        uint64_t c = 0;
        for (int64_t b = 0; b < blocks; ++b) {
            acc = acc + part_mass[b * E + e];
            c += part_counts[b * E + e];
        }
        mass_sh[e] = acc;
        counts_sh[e] = static_cast<float>(c);
        mass[e] = acc;
        counts[e] = static_cast<float>(c);
    }
    if (tid == 0) {
        uint64_t v = 0;
        for (int64_t b = 0; b < blocks; ++b) v += part_valid[b];
        valid_sh = static_cast<float>(v);
        valid_count[0] = valid_sh;
    }
    __syncthreads();
    if (tid == 0 && loss != nullptr) loss[0] = balance_loss_of(mass_sh, counts_sh, valid_sh, E);
}

__global__ void balance_loss_kernel(const float* __restrict__ mass, const float* __restrict__ counts,
                                    const float* __restrict__ valid_count, int64_t E, float* __restrict__ loss) {
    if (threadIdx.x == 0 && blockIdx.x == 0) loss[0] = balance_loss_of(mass, counts, valid_count[0], E);
}

template <typename I>
__global__ void check_assignments_kernel(const I* __restrict__ a, const uint8_t* __restrict__ valid,
                                         int32_t* __restrict__ flags, int64_t T, int64_t k, int64_t E) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T || !valid[t]) return;
    const I* row = a + t * k;
    bool out_of_range = false, dup = false;
    for (int64_t s = 0; s < k; ++s) {
        const int64_t e = static_cast<int64_t>(row[s]);
        out_of_range |= (e < 0 || e >= E);
        for (int64_t r = 0; r < s; ++r) dup |= (static_cast<int64_t>(row[r]) == e);
    }
    if (out_of_range) atomicOr(flags, 1);
    if (dup) atomicOr(flags + 1, 1);
}

constexpr int kCountThreads = 256;
constexpr int kCountLdsBins = 4096;

template <typename I>
__global__ __launch_bounds__(kCountThreads) void expert_counts_kernel(
    const I* __restrict__ a, const uint8_t* __restrict__ valid, unsigned long long* __restrict__ counts,
    int64_t T, int64_t k, int64_t E) {
    __shared__ uint32_t hist[kCountLdsBins];
    const bool use_lds = E <= kCountLdsBins;
    if (use_lds) {
        for (int64_t e = threadIdx.x; e < E; e += kCountThreads) hist[e] = 0;
        __syncthreads();
    }
    const int64_t pairs = T * k;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kCountThreads;
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * kCountThreads + threadIdx.x; p < pairs; p += stride) {
        const int64_t t = p / k;
        const int64_t e = static_cast<int64_t>(a[p]);
        if (valid[t] && e >= 0 && e < E) {
            if (use_lds) atomicAdd(&hist[e], 1u);
            else atomicAdd(&counts[e], 1ull);
        }
    }
    if (use_lds) {
        __syncthreads();
        for (int64_t e = threadIdx.x; e < E; e += kCountThreads)
            if (hist[e]) atomicAdd(&counts[e], static_cast<unsigned long long>(hist[e]));
    }
}

__global__ void zero_i64_kernel(int64_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_moe_route_hash(const void* token_ids, const void* previous_token_ids,
                                    const uint8_t* valid_mask, int id_dtype, int64_t* assignments,
                                    int32_t* duplicate_flag, int64_t tokens, int64_t expert_count,
                                    int64_t top_k, koemi_stream_t stream) {
    if (tokens < 0) return fail(KOEMI_ERR_INVALID, "token count must be non-negative");
    if (expert_count < 1 || top_k < 1 || top_k > expert_count)
        return fail(KOEMI_ERR_INVALID, "route needs 1 <= top_k <= expert_count");
    if (!index_dtype(id_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "token ids must be int32 or int64");
    if (tokens == 0) return KOEMI_OK;
    if (!token_ids || !previous_token_ids || !valid_mask || !assignments)
        return fail(KOEMI_ERR_INVALID, "route received a null pointer");
    const dim3 grid(grid_for(tokens, 256)), block(256);
    hipStream_t s = as_stream(stream);
    if (id_dtype == KOEMI_I32)
        hipLaunchKernelGGL(route_hash_kernel<int32_t>, grid, block, 0, s, static_cast<const int32_t*>(token_ids),
                           static_cast<const int32_t*>(previous_token_ids), valid_mask, assignments, duplicate_flag,
                           tokens, expert_count, top_k);
    else
        hipLaunchKernelGGL(route_hash_kernel<int64_t>, grid, block, 0, s, static_cast<const int64_t*>(token_ids),
                           static_cast<const int64_t*>(previous_token_ids), valid_mask, assignments, duplicate_flag,
                           tokens, expert_count, top_k);
    return check_launch("koemi_moe_route_hash");
}

extern "C" int koemi_moe_route_modulo(const void* token_ids, const uint8_t* valid_mask, int id_dtype,
                                      int64_t* assignments, int64_t tokens, int64_t expert_count, int64_t top_k,
                                      koemi_stream_t stream) {
    if (tokens < 0) return fail(KOEMI_ERR_INVALID, "token count must be non-negative");
    if (expert_count < 1 || top_k < 1 || top_k > expert_count)
        return fail(KOEMI_ERR_INVALID, "route needs 1 <= top_k <= expert_count");
    if (!index_dtype(id_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "token ids must be int32 or int64");
    if (tokens == 0) return KOEMI_OK;
    if (!token_ids || !valid_mask || !assignments) return fail(KOEMI_ERR_INVALID, "route received a null pointer");
    const dim3 grid(grid_for(tokens, 256)), block(256);
    hipStream_t s = as_stream(stream);
    if (id_dtype == KOEMI_I32)
        hipLaunchKernelGGL(route_modulo_kernel<int32_t>, grid, block, 0, s, static_cast<const int32_t*>(token_ids),
                           valid_mask, assignments, tokens, expert_count, top_k);
    else
        hipLaunchKernelGGL(route_modulo_kernel<int64_t>, grid, block, 0, s, static_cast<const int64_t*>(token_ids),
                           valid_mask, assignments, tokens, expert_count, top_k);
    return check_launch("koemi_moe_route_modulo");
}

extern "C" int koemi_moe_route_learned(const float* router_logits, const uint8_t* valid_mask,
                                       int64_t* assignments, float* weights, int64_t tokens,
                                       int64_t expert_count, int64_t top_k, koemi_stream_t stream) {
    if (tokens < 0) return fail(KOEMI_ERR_INVALID, "token count must be non-negative");
    if (expert_count < 1 || top_k < 1 || top_k > expert_count)
        return fail(KOEMI_ERR_INVALID, "learned route needs 1 <= top_k <= expert_count");
    if (expert_count > 1024) return fail(KOEMI_ERR_UNSUPPORTED, "learned route supports at most 1024 experts");
    if (tokens == 0) return KOEMI_OK;
    if (!router_logits || !valid_mask || !assignments || !weights)
        return fail(KOEMI_ERR_INVALID, "learned route received a null pointer");
    hipLaunchKernelGGL(route_learned_kernel, dim3(grid_for(tokens, 256)), dim3(256), 0, as_stream(stream),
                       router_logits, valid_mask, assignments, weights, tokens, expert_count, top_k);
    return check_launch("koemi_moe_route_learned");
}

extern "C" size_t koemi_moe_route_learned_stats_workspace_bytes(int64_t tokens, int64_t expert_count) {
    if (tokens < 0 || expert_count < 1) return 0;
    const int64_t blocks = (tokens + kStatThreads - 1) / kStatThreads;
    return static_cast<size_t>(blocks) * static_cast<size_t>(2 * expert_count + 1) * 4u;
}

extern "C" int koemi_moe_route_learned_stats(const float* router_logits, const uint8_t* valid_mask,
                                             int64_t* assignments, float* weights, float* probability_mass,
                                             float* assignment_counts, float* valid_count, float* balance_loss,
                                             int64_t tokens, int64_t expert_count, int64_t top_k, void* workspace,
                                             size_t workspace_bytes, koemi_stream_t stream) {
    if (tokens < 0) return fail(KOEMI_ERR_INVALID, "token count must be non-negative");
    if (expert_count < 1 || top_k < 1 || top_k > expert_count)
        return fail(KOEMI_ERR_INVALID, "learned route needs 1 <= top_k <= expert_count");
    if (expert_count > kStatMaxExperts)
        return fail(KOEMI_ERR_UNSUPPORTED, "learned route supports at most %d experts", kStatMaxExperts);
    if (!probability_mass || !assignment_counts || !valid_count)
        return fail(KOEMI_ERR_INVALID, "learned route statistics received a null pointer");
    const int64_t blocks = (tokens + kStatThreads - 1) / kStatThreads;
    hipStream_t s = as_stream(stream);
    if (tokens > 0) {
        if (!router_logits || !valid_mask || !assignments || !weights || !workspace)
            return fail(KOEMI_ERR_INVALID, "learned route received a null pointer");
        const size_t need = koemi_moe_route_learned_stats_workspace_bytes(tokens, expert_count);
        if (workspace_bytes < need)
            return fail(KOEMI_ERR_INVALID, "learned route statistics workspace too small: need %zu bytes", need);
        if (blocks > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "learned route: too many tokens");
    }
    float* part_mass = static_cast<float*>(workspace);
    uint32_t* part_counts = reinterpret_cast<uint32_t*>(part_mass + blocks * expert_count);
    uint32_t* part_valid = part_counts + blocks * expert_count;
    if (tokens > 0) {
        hipLaunchKernelGGL(route_learned_stats_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kStatThreads), 0, s,
                           router_logits, valid_mask, assignments, weights, tokens, expert_count, top_k, part_mass,
                           part_counts, part_valid);
        if (int st = check_launch("koemi_moe_route_learned_stats")) return st;
    }
    hipLaunchKernelGGL(router_stats_finish_kernel, dim3(1), dim3(kStatThreads), 0, s, part_mass, part_counts,
                       part_valid, blocks, expert_count, probability_mass, assignment_counts, valid_count,
                       balance_loss);
    return check_launch("koemi_moe_route_learned_stats (finish)");
}

extern "C" int koemi_moe_router_balance_loss(const float* probability_mass, const float* assignment_counts,
                                             const float* valid_count, int64_t expert_count, float* balance_loss,
                                             koemi_stream_t stream) {
    if (expert_count < 1) return fail(KOEMI_ERR_INVALID, "balance loss needs at least one expert");
    if (!probability_mass || !assignment_counts || !valid_count || !balance_loss)
        return fail(KOEMI_ERR_INVALID, "balance loss received a null pointer");
    hipLaunchKernelGGL(balance_loss_kernel, dim3(1), dim3(64), 0, as_stream(stream), probability_mass,
                       assignment_counts, valid_count, expert_count, balance_loss);
    return check_launch("koemi_moe_router_balance_loss");
}

extern "C" int koemi_moe_check_assignments(const void* assignments, int assignment_dtype,
                                           const uint8_t* valid_mask, int32_t* flags, int64_t tokens,
                                           int64_t top_k, int64_t expert_count, koemi_stream_t stream) {
    if (tokens < 0 || top_k < 1 || expert_count < 1) return fail(KOEMI_ERR_INVALID, "invalid assignment check sizes");
    if (!index_dtype(assignment_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "assignments must be int32 or int64");
    if (tokens == 0) return KOEMI_OK;
    if (!assignments || !valid_mask || !flags) return fail(KOEMI_ERR_INVALID, "assignment check received a null pointer");
    const dim3 grid(grid_for(tokens, 256)), block(256);
    hipStream_t s = as_stream(stream);
    if (assignment_dtype == KOEMI_I32)
        hipLaunchKernelGGL(check_assignments_kernel<int32_t>, grid, block, 0, s, static_cast<const int32_t*>(assignments),
                           valid_mask, flags, tokens, top_k, expert_count);
    else
        hipLaunchKernelGGL(check_assignments_kernel<int64_t>, grid, block, 0, s, static_cast<const int64_t*>(assignments),
                           valid_mask, flags, tokens, top_k, expert_count);
    return check_launch("koemi_moe_check_assignments");
}

extern "C" int koemi_moe_expert_counts(const void* assignments, int assignment_dtype,
                                       const uint8_t* valid_mask, int64_t* counts, int64_t tokens,
                                       int64_t top_k, int64_t expert_count, koemi_stream_t stream) {
    if (tokens < 0 || top_k < 1 || expert_count < 1) return fail(KOEMI_ERR_INVALID, "invalid expert count sizes");
    if (!index_dtype(assignment_dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "assignments must be int32 or int64");
    if (!counts) return fail(KOEMI_ERR_INVALID, "expert counts received a null pointer");
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(zero_i64_kernel, dim3(grid_for(expert_count, 256)), dim3(256), 0, s, counts, expert_count);
    int st = check_launch("koemi_moe_expert_counts");
    if (st != KOEMI_OK || tokens == 0) return st;
    if (!assignments || !valid_mask) return fail(KOEMI_ERR_INVALID, "expert counts received a null pointer");
    int64_t blocks = (tokens * top_k + kCountThreads * 16 - 1) / (kCountThreads * 16);
    if (blocks < 1) blocks = 1;
    if (blocks > 1024) blocks = 1024;
    unsigned long long* c = reinterpret_cast<unsigned long long*>(counts);
    if (assignment_dtype == KOEMI_I32)
        hipLaunchKernelGGL(expert_counts_kernel<int32_t>, dim3(static_cast<unsigned>(blocks)), dim3(kCountThreads), 0, s,
                           static_cast<const int32_t*>(assignments), valid_mask, c, tokens, top_k, expert_count);
    else
        hipLaunchKernelGGL(expert_counts_kernel<int64_t>, dim3(static_cast<unsigned>(blocks)), dim3(kCountThreads), 0, s,
                           static_cast<const int64_t*>(assignments), valid_mask, c, tokens, top_k, expert_count);
    return check_launch("koemi_moe_expert_counts");
}
