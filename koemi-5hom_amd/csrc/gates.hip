// Bounded recurrent gates for gfx950.
//
// Reference: model/memory.py:14-30 (BoundedRecurrentState.gates) and the
// masking of network.py:306-309:
//
//   retention = sigmoid(u W_r^T + b_r)
//   a = 2^-8 + ((1 - 2^-8) - 2^-8) * retention        (in [2^-8, 1 - 2^-8])
//   b = (1 - a) * tanh(u W_c^T + b_c)
//   invalid positions (valid mask given and false): a = 1, b = 0
//
// The two width x width products are plain GEMMs and run on rocBLAS (fp32
// accumulation, fp32 results in the workspace); one HIP kernel then applies
// the biases, the bounded sigmoid, tanh and the mask and writes a and b in the
// input dtype, reading each fp32 product once (16-byte loads, four columns per
// thread). koemi_recurrent_scan (fp32) hands the two products straight to the
// affine-scan kernel, which applies the same expressions in registers, so a
// and b never reach memory.
#include "common.hpp"

#include <rocblas/rocblas.h>

#include <mutex>

namespace koemi {

// The rocBLAS handle of a device (blas.hip); callers hold g_blas_mutex.
rocblas_handle blas_handle(int device);
extern std::mutex g_blas_mutex;
// The fused gates + scan kernel (affine_scan.hip).
int launch_gated_scan(const float* zr, const float* zc, int64_t stride, const float* retention_bias,
                      const float* candidate_bias, const uint8_t* valid, const float* h0, float* h, void* h16,
                      int64_t h16_stride, int64_t B, int64_t L, int64_t F, hipStream_t stream, void* workspace,
                      size_t workspace_bytes);

namespace {


template <typename T>
__global__ __launch_bounds__(256) void gates_epilogue_kernel(
    const float* __restrict__ zr, const float* __restrict__ zc, const T* __restrict__ br, const T* __restrict__ bc,
    const uint8_t* __restrict__ valid, T* __restrict__ a_out, T* __restrict__ b_out, int64_t rows, int64_t D) {
    const int64_t quads = D / 4;
    const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (q >= rows * quads) return;
    const int64_t row = q / quads;
    const int64_t c0 = (q - row * quads) * 4;
    const float4 r4 = *reinterpret_cast<const float4*>(zr + row * D + c0);
    const float4 z4 = *reinterpret_cast<const float4*>(zc + row * D + c0);
    const float r[4] = {r4.x, r4.y, r4.z, r4.w}, z[4] = {z4.x, z4.y, z4.z, z4.w};
    const bool keep = valid == nullptr || valid[row] != 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float a = kGateMinRetention + kGateRetentionSpan * gate_sigmoid(r[c] + to_f32(br[c0 + c]));
        const float b = (1.0f - a) * gate_tanh(z[c] + to_f32(bc[c0 + c]));
        a_out[row * D + c0 + c] = from_f32<T>(keep ? a : 1.0f);
        b_out[row * D + c0 + c] = from_f32<T>(keep ? b : 0.0f);
    }
}

rocblas_datatype gates_blas_type(int dtype) {
    switch (dtype) {
        case KOEMI_F16: return rocblas_datatype_f16_r;
        case KOEMI_BF16: return rocblas_datatype_bf16_r;
        default: return rocblas_datatype_f32_r;
    }
}

size_t gates_workspace(int64_t rows, int64_t D) {
    const size_t one = (static_cast<size_t>(rows) * static_cast<size_t>(D) * sizeof(float) + 255) & ~size_t(255);
    return 2 * one;
}

// zr = u W_r^T, zc = u W_c^T (row-major [rows, D], fp32) on rocBLAS: in its
// column-major terms Z' (D x rows) = W'^T (D x D) . u' (D x rows).
int gate_products(const void* input, const void* retention_weight, const void* candidate_weight, float* zr,
                  float* zc, int64_t rows, int64_t width, int dtype, hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(KOEMI_ERR_LAUNCH, "recurrent gates: no device");
    std::lock_guard<std::mutex> lock(g_blas_mutex);
    rocblas_handle h = blas_handle(dev);
    if (!h) return fail(KOEMI_ERR_LAUNCH, "recurrent gates: no rocBLAS handle");
    if (rocblas_set_stream(h, s) != rocblas_status_success ||
        rocblas_set_pointer_mode(h, rocblas_pointer_mode_host) != rocblas_status_success)
        return fail(KOEMI_ERR_LAUNCH, "recurrent gates: rocblas stream setup failed");
    const rocblas_datatype t = gates_blas_type(dtype);
    const rocblas_int d = static_cast<rocblas_int>(width), n = static_cast<rocblas_int>(rows);
    const float one = 1.0f, zero = 0.0f;
    for (int g = 0; g < 2; ++g) {
        const void* w = g == 0 ? retention_weight : candidate_weight;
        float* z = g == 0 ? zr : zc;
        const rocblas_status st = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, d, n, d, &one,
                                                  w, t, d, input, t, d, &zero, z, rocblas_datatype_f32_r, d, z,
                                                  rocblas_datatype_f32_r, d, rocblas_datatype_f32_r,
                                                  rocblas_gemm_algo_standard, 0, 0);
        if (st != rocblas_status_success)
            return fail(KOEMI_ERR_LAUNCH, "recurrent gates: rocblas_gemm_ex failed (%s)", rocblas_status_to_string(st));
    }
    return KOEMI_OK;
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" size_t koemi_recurrent_gates_workspace_bytes(int64_t rows, int64_t width) {
    if (rows < 0 || width < 1) return 0;
    return gates_workspace(rows, width);
}

extern "C" int koemi_recurrent_gates(const void* input, const void* retention_weight, const void* retention_bias,
                                     const void* candidate_weight, const void* candidate_bias, const uint8_t* valid,
                                     void* retention_out, void* increment_out, int64_t rows, int64_t width, int dtype,
                                     void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (rows < 0 || width < 1) return fail(KOEMI_ERR_INVALID, "recurrent gates need non-negative rows and positive width");
    if (!float_dtype(dtype)) return fail(KOEMI_ERR_UNSUPPORTED, "recurrent gates do not support dtype %s", dtype_name(dtype));
    if (width % 4 != 0) return fail(KOEMI_ERR_UNSUPPORTED, "recurrent gates need width % 4 == 0");
    if (rows == 0) return KOEMI_OK;
    if (rows > 0x7fffffffLL || width > 0x7fffffffLL / 4)
        return fail(KOEMI_ERR_UNSUPPORTED, "recurrent gates sizes exceed 32-bit GEMM dimensions");
    if (!input || !retention_weight || !retention_bias || !candidate_weight || !candidate_bias || !retention_out ||
        !increment_out)
        return fail(KOEMI_ERR_INVALID, "recurrent gates received a null pointer");
    const size_t need = gates_workspace(rows, width);
    if (!workspace || workspace_bytes < need)
        return fail(KOEMI_ERR_INVALID, "recurrent gates workspace too small: need %zu bytes", need);
    float* zr = static_cast<float*>(workspace);
    float* zc = reinterpret_cast<float*>(static_cast<char*>(workspace) + need / 2);
    const hipStream_t s = as_stream(stream);

    {
        const int st = gate_products(input, retention_weight, candidate_weight, zr, zc, rows, width, dtype, s);
        if (st != KOEMI_OK) return st;
    }
    const int64_t quads = rows * (width / 4);
    const dim3 grid(static_cast<unsigned>((quads + 255) / 256)), block(256);
    switch (dtype) {
        case KOEMI_F32:
            hipLaunchKernelGGL(gates_epilogue_kernel<float>, grid, block, 0, s, zr, zc,
                               static_cast<const float*>(retention_bias), static_cast<const float*>(candidate_bias),
                               valid, static_cast<float*>(retention_out), static_cast<float*>(increment_out), rows, width);
            break;
        case KOEMI_F16:
            hipLaunchKernelGGL(gates_epilogue_kernel<f16>, grid, block, 0, s, zr, zc,
                               static_cast<const f16*>(retention_bias), static_cast<const f16*>(candidate_bias), valid,
                               static_cast<f16*>(retention_out), static_cast<f16*>(increment_out), rows, width);
            break;
        default:
            hipLaunchKernelGGL(gates_epilogue_kernel<bf16>, grid, block, 0, s, zr, zc,
                               static_cast<const bf16*>(retention_bias), static_cast<const bf16*>(candidate_bias),
                               valid, static_cast<bf16*>(retention_out), static_cast<bf16*>(increment_out), rows, width);
    }
    return check_launch("koemi_recurrent_gates");
}

extern "C" int koemi_recurrent_scan(const float* input, const float* retention_weight, const float* retention_bias,
                                    const float* candidate_weight, const float* candidate_bias, const uint8_t* valid,
                                    const float* initial, float* states, int64_t batch, int64_t length, int64_t width,
                                    void* workspace, size_t workspace_bytes, koemi_stream_t stream) {
    if (batch < 0 || length < 0 || width < 1)
        return fail(KOEMI_ERR_INVALID, "recurrent scan needs non-negative batch and length and a positive width");
    if (width % 4 != 0) return fail(KOEMI_ERR_UNSUPPORTED, "recurrent scan needs width % 4 == 0");
    const int64_t rows = batch * length;
    if (rows == 0) return KOEMI_OK;
    if (rows > 0x7fffffffLL || width > 0x7fffffffLL / 4)
        return fail(KOEMI_ERR_UNSUPPORTED, "recurrent scan sizes exceed 32-bit GEMM dimensions");
    if (batch * ((width + kWave - 1) / kWave) > 0x7fffffffLL)
        return fail(KOEMI_ERR_UNSUPPORTED, "recurrent scan grid too large");
    if (!input || !retention_weight || !retention_bias || !candidate_weight || !candidate_bias || !initial || !states)
        return fail(KOEMI_ERR_INVALID, "recurrent scan received a null pointer");
    const size_t need = gates_workspace(rows, width);
    if (!workspace || workspace_bytes < need)
        return fail(KOEMI_ERR_INVALID, "recurrent scan workspace too small: need %zu bytes", need);
    float* zr = static_cast<float*>(workspace);
    float* zc = reinterpret_cast<float*>(static_cast<char*>(workspace) + need / 2);
    const hipStream_t s = as_stream(stream);
    int st = gate_products(input, retention_weight, candidate_weight, zr, zc, rows, width, KOEMI_F32, s);
    if (st != KOEMI_OK) return st;
    return launch_gated_scan(zr, zc, width, retention_bias, candidate_bias, valid, initial, states, nullptr, width,
                             batch, length, width, s, nullptr, 0);
}
