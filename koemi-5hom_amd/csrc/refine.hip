// The refine memory of the herm ablation, the parts besides its associative
// scan (which assoc_memory.hip runs): the novelty output of the local read and
// the refine gate.
//
// Reference: LocalKeyValueMemory.read_window's novelty (model/memory.py:
// 354-361: the largest cosine similarity of each query with the keys of its
// sliding window, novelty = clamp(1 - largest, 0, 1), 1 with no eligible
// slot) and KoemiModel.refine_memory (network.py:714-721: memory value =
// fast + sigmoid(W_g [working; fast; refine; local] + b_g) * refine), torch
// composites in the reference. Both are row-local; one wave per query (the
// novelty's at most `window` dot products over the width) or per position
// (the gate's dot product over four widths, then the mix).
#include "common.hpp"

namespace koemi {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Query t of window row r: slot s of [carried (C) ; window (L)] is eligible
// when C + t - window <= s < C + t and its valid byte is set (the local
// read's sliding_window_mask, memory.py:364-383). similarity = k . q /
// (max(|k|, 1e-12) max(|q|, 1e-12)) (functional.normalize on both).
template <typename KT>
__global__ __launch_bounds__(256) void local_novelty_kernel(
    const float* __restrict__ carried_keys, const uint8_t* __restrict__ carried_valid, const KT* __restrict__ keys,
    int64_t key_stride, const uint8_t* __restrict__ key_valid, const float* __restrict__ queries, int64_t q_stride,
    float* __restrict__ novelty, int64_t rows, int64_t C, int64_t L, int64_t D, int64_t window) {
    const int lane = lane_id();
    const int64_t job = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;  // (row, query)
    if (job >= rows * L) return;
    const int64_t r = job / L, t = job - r * L;
    const float* q = queries + job * q_stride;
    float qq = 0.0f;
    for (int64_t d = lane; d < D; d += kWave) qq = fmaf(q[d], q[d], qq);
    const float qn = fmaxf(sqrtf(wave_sum(qq)), 1e-12f);
    const int64_t own = C + t;
    float best = -INFINITY;
    bool any = false;
    for (int64_t s = own - window > 0 ? own - window : 0; s < own; ++s) {  // wave-uniform
        const bool carried = s < C;
        if (!(carried ? carried_valid[r * C + s] : key_valid[r * L + (s - C)])) continue;
        float dot = 0.0f, kk = 0.0f;
        if (carried) {
            const float* k = carried_keys + (r * C + s) * D;
            for (int64_t d = lane; d < D; d += kWave) {
                dot = fmaf(k[d], q[d], dot);
                kk = fmaf(k[d], k[d], kk);
            }
        } else {
            const KT* k = keys + (r * L + (s - C)) * key_stride;
            for (int64_t d = lane; d < D; d += kWave) {
                const float x = to_f32(k[d]);
                dot = fmaf(x, q[d], dot);
                kk = fmaf(x, x, kk);
            }
        }
        dot = wave_sum(dot);
        kk = wave_sum(kk);
        best = fmaxf(best, dot / (fmaxf(sqrtf(kk), 1e-12f) * qn));
        any = true;
    }
    if (lane == 0) novelty[job] = any ? fminf(fmaxf(1.0f - best, 0.0f), 1.0f) : 1.0f;
}

// Position p: pre = sum_k x_k w_k + b over x = [working; fast; refine;
// local] (LOW: every x_k and w_k rounded to bf16, fp32 accumulation, the sum
// rounded to bf16 after the bias: nn.Linear under bf16 autocast), g =
// sigmoid(pre), out = fast + g refine.
template <typename LT, typename WT, typename OT, bool LOW>
__global__ __launch_bounds__(256) void refine_gate_kernel(
    const float* __restrict__ ws, int64_t ws_stride, const float* __restrict__ fast, int64_t fast_stride,
    const float* __restrict__ refine, int64_t refine_stride, const LT* __restrict__ local, int64_t local_stride,
    const WT* __restrict__ weight, const float* __restrict__ bias, OT* __restrict__ out, int64_t out_stride,
    int64_t rows, int64_t D) {
    const int lane = lane_id();
    const int64_t p = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (p >= rows) return;
    auto rnd = [](float x) { return LOW ? static_cast<float>(static_cast<bf16>(x)) : x; };
    const float* w0 = ws + p * ws_stride;
    const float* f0 = fast + p * fast_stride;
    const float* r0 = refine + p * refine_stride;
    const LT* l0 = local + p * local_stride;
    float acc = 0.0f;
    for (int64_t d = lane; d < D; d += kWave) {
        acc = fmaf(rnd(w0[d]), to_f32(weight[d]), acc);
        acc = fmaf(rnd(f0[d]), to_f32(weight[D + d]), acc);
        acc = fmaf(rnd(r0[d]), to_f32(weight[2 * D + d]), acc);
        acc = fmaf(rnd(to_f32(l0[d])), to_f32(weight[3 * D + d]), acc);
    }
    const float pre = rnd(wave_sum(acc) + bias[0]);
    const float g = 1.0f / (1.0f + expf(-pre));
    OT* o = out + p * out_stride;
    for (int64_t d = lane; d < D; d += kWave) o[d] = from_f32<OT>(fmaf(g, r0[d], f0[d]));
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_local_novelty(const float* carried_keys, const uint8_t* carried_valid, const void* keys,
                                   int key_dtype, int64_t key_row_stride, const uint8_t* key_valid,
                                   const float* queries, int64_t query_row_stride, float* novelty, int64_t rows,
                                   int64_t capacity, int64_t length, int64_t width, int64_t window,
                                   koemi_stream_t stream) {
    if (rows < 0 || capacity < 0 || length < 0 || width < 1 || window < 1)
        return fail(KOEMI_ERR_INVALID, "local novelty needs non-negative rows, capacity and length, positive width and "
                    "window");
    if (key_dtype != KOEMI_F32 && key_dtype != KOEMI_BF16)
        return fail(KOEMI_ERR_UNSUPPORTED, "local novelty keys must be float32 or bfloat16");
    if (key_row_stride == 0) key_row_stride = width;
    if (query_row_stride == 0) query_row_stride = width;
    if (key_row_stride < width || query_row_stride < width)
        return fail(KOEMI_ERR_INVALID, "local novelty row strides must not be below the width");
    if (rows * length == 0) return KOEMI_OK;
    if (!keys || !key_valid || !queries || !novelty || (capacity > 0 && (!carried_keys || !carried_valid)))
        return fail(KOEMI_ERR_INVALID, "local novelty received a null pointer");
    const int64_t jobs = rows * length;
    if ((jobs + 3) / 4 > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "local novelty grid too large");
    const dim3 grid(static_cast<unsigned>((jobs + 3) / 4));
    hipStream_t s = as_stream(stream);
    if (key_dtype == KOEMI_BF16)
        hipLaunchKernelGGL(local_novelty_kernel<bf16>, grid, dim3(256), 0, s, carried_keys, carried_valid,
                           static_cast<const bf16*>(keys), key_row_stride, key_valid, queries, query_row_stride, novelty,
                           rows, capacity, length, width, window);
    else
        hipLaunchKernelGGL(local_novelty_kernel<float>, grid, dim3(256), 0, s, carried_keys, carried_valid,
                           static_cast<const float*>(keys), key_row_stride, key_valid, queries, query_row_stride,
                           novelty, rows, capacity, length, width, window);
    return check_launch("koemi_local_novelty");
}

extern "C" int koemi_herm_refine_gate(const float* working, int64_t working_row_stride, const float* fast,
                                      int64_t fast_row_stride, const float* refine, int64_t refine_row_stride,
                                      const void* local, int local_dtype, int64_t local_row_stride,
                                      const void* weight, int weight_dtype, const float* bias, int round_bf16,
                                      void* out, int out_dtype, int64_t out_row_stride, int64_t rows, int64_t width,
                                      koemi_stream_t stream) {
    if (rows < 0 || width < 1) return fail(KOEMI_ERR_INVALID, "refine gate needs non-negative rows and positive width");
    auto ok_dtype = [](int d) { return d == KOEMI_F32 || d == KOEMI_BF16; };
    if (!ok_dtype(local_dtype) || !ok_dtype(weight_dtype) || !ok_dtype(out_dtype))
        return fail(KOEMI_ERR_UNSUPPORTED, "refine gate tensors must be float32 or bfloat16");
    int64_t* strides[] = {&working_row_stride, &fast_row_stride, &refine_row_stride, &local_row_stride,
                          &out_row_stride};
    for (int64_t* st : strides) {
        if (*st == 0) *st = width;
        if (*st < width) return fail(KOEMI_ERR_INVALID, "refine gate row strides must not be below the width");
    }
    if (rows == 0) return KOEMI_OK;
    if (!working || !fast || !refine || !local || !weight || !bias || !out)
        return fail(KOEMI_ERR_INVALID, "refine gate received a null pointer");
    if ((rows + 3) / 4 > 0x7fffffffLL) return fail(KOEMI_ERR_UNSUPPORTED, "refine gate grid too large");
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
    hipStream_t s = as_stream(stream);
    auto go = [&](auto lt, auto wt, auto ot, auto low) {
        using LT = decltype(lt);
        using WT = decltype(wt);
        using OT = decltype(ot);
        hipLaunchKernelGGL((refine_gate_kernel<LT, WT, OT, decltype(low)::value>), grid, dim3(256), 0, s, working,
                           working_row_stride, fast, fast_row_stride, refine, refine_row_stride,
                           static_cast<const LT*>(local), local_row_stride, static_cast<const WT*>(weight), bias,
                           static_cast<OT*>(out), out_row_stride, rows, width);
    };
    // bf16 stacks (bf16 weight, rounding on): bf16 or fp32 local read, bf16 or
    // fp32 output; fp32 stacks: everything fp32
    if (round_bf16) {
        if (weight_dtype != KOEMI_BF16)
            return fail(KOEMI_ERR_UNSUPPORTED, "the rounding refine gate takes a bfloat16 weight");
        if (local_dtype == KOEMI_BF16) {
            if (out_dtype == KOEMI_BF16) go(bf16{}, bf16{}, bf16{}, std::true_type{});
            else go(bf16{}, bf16{}, float{}, std::true_type{});
        } else {
            if (out_dtype == KOEMI_BF16) go(float{}, bf16{}, bf16{}, std::true_type{});
            else go(float{}, bf16{}, float{}, std::true_type{});
        }
    } else {
        if (weight_dtype != KOEMI_F32 || local_dtype != KOEMI_F32 || out_dtype != KOEMI_F32)
            return fail(KOEMI_ERR_UNSUPPORTED, "the fp32 refine gate takes float32 tensors");
        go(float{}, float{}, float{}, std::false_type{});
    }
    return check_launch("koemi_herm_refine_gate");
}
