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
// The two products are plain batched GEMMs and run on rocBLAS (fp32
// accumulation), each as two strided-batched calls (the carried and the
// window part of the key axis) that address the caller's tensors in place, so
// nothing is concatenated. The masked softmax between them is a HIP kernel: a
// wave per query row builds the eligibility from the valid/admission bytes and
// the positions, takes the row maximum and the exponential sum in fp32, and
// writes the weights (in the input dtype, which the second product reads).
// rocBLAS is column-major: a row-major [rows, cols] matrix is its [cols, rows]
// column-major view, so score^T = K'^T Q' and out' = V' P'.
#include "common.hpp"

#include <rocblas/rocblas.h>

#include <cmath>
#include <mutex>

namespace koemi {

// The rocBLAS handle of a device (blas.hip); callers hold g_blas_mutex.
rocblas_handle blas_handle(int device);
extern std::mutex g_blas_mutex;

namespace {

constexpr int kSoftmaxWaves = 4;

template <typename T>
__global__ __launch_bounds__(kWave * kSoftmaxWaves) void masked_softmax_kernel(
    const float* __restrict__ score, const uint8_t* __restrict__ carried_valid, const uint8_t* __restrict__ admission,
    T* __restrict__ weight, int64_t B, int64_t S, int64_t L) {
    const int lane = lane_id();
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kSoftmaxWaves + threadIdx.x / kWave;  // b * L + t
    if (row >= B * L) return;
    const int64_t b = row / L, t = row % L;
    const int64_t K = S + L;
    const float* x = score + row * K;
    T* w = weight + row * K;
    auto eligible = [&](int64_t s) -> bool {
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
    if (dtype == KOEMI_F32) {
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

extern "C" int koemi_salient_read(const void* carried_keys, const void* carried_values, const uint8_t* carried_valid,
                                  const void* keys, const void* values, const uint8_t* admission, const void* queries,
                                  void* out, int64_t batch, int64_t carried, int64_t length, int64_t width, int dtype,
                                  void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || carried < 0 || length < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "salient read needs non-negative batch, carried and length and positive width");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "salient read does not support dtype %s", dtype_name(dtype));
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
    char* base = static_cast<char*>(workspace);
    float* score = reinterpret_cast<float*>(base + ws.score_off);
    void* weight = base + ws.weight_off;
    const hipStream_t s = as_stream(stream);

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
                               static_cast<float*>(weight), batch, carried, length);
            break;
        case KOEMI_F16:
            hipLaunchKernelGGL(masked_softmax_kernel<f16>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<f16*>(weight), batch, carried, length);
            break;
        default:
            hipLaunchKernelGGL(masked_softmax_kernel<bf16>, grid, block, 0, s, score, carried_valid, admission,
                               static_cast<bf16*>(weight), batch, carried, length);
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
