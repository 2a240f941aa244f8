// Streaming-read floor: the time a plain read of N bytes takes on this chip
// with a given launch shape, for judging the memory-bound kernels (the
// surprise rows and the RMSNorm-SiLU of configuration 2 move 34 and 67 MB per
// call) against what a read of that size can reach here at all. Measurement
// only; nothing on the hot path calls it.
//
// Each thread issues U 16-byte loads (all in flight before the first use) per
// pass of a grid-stride loop and folds them into one sum, which is stored only
// if it equals a value the benchmark never produces, so the loads cannot be
// dropped and the stores cost nothing.
#include "common.hpp"

namespace koemi {
namespace {

template <int U>
__global__ void stream_read_kernel(const float4* __restrict__ src, int64_t n16, float* __restrict__ sink) {
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    float acc = 0.0f;
    for (int64_t i = tid; i < n16; i += stride * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = i + u * stride;
            v[u] = j < n16 ? src[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    if (acc == -1.2345678e30f) sink[tid] = acc;
}

}  // namespace
}  // namespace koemi

using namespace koemi;

extern "C" int koemi_stream_read(const void* src, int64_t bytes, int unroll, int block, int64_t grid, float* sink,
                                 koemi_stream_t stream) {
    if (bytes < 0 || bytes % 16 || grid < 1 || grid > 0x7fffffffLL || (block != 64 && block != 128 && block != 256 &&
                                                                       block != 512 && block != 1024))
        return fail(KOEMI_ERR_INVALID, "stream read needs bytes % 16 == 0, grid >= 1 and a block of 64..1024 threads");
    if (bytes == 0) return KOEMI_OK;
    if (!src || !sink) return fail(KOEMI_ERR_INVALID, "stream read received a null pointer");
    const dim3 g(static_cast<uint32_t>(grid)), b(static_cast<uint32_t>(block));
    hipStream_t s = as_stream(stream);
    const float4* p = static_cast<const float4*>(src);
    const int64_t n16 = bytes / 16;
    switch (unroll) {
        case 1: hipLaunchKernelGGL(stream_read_kernel<1>, g, b, 0, s, p, n16, sink); break;
        case 2: hipLaunchKernelGGL(stream_read_kernel<2>, g, b, 0, s, p, n16, sink); break;
        case 4: hipLaunchKernelGGL(stream_read_kernel<4>, g, b, 0, s, p, n16, sink); break;
        case 8: hipLaunchKernelGGL(stream_read_kernel<8>, g, b, 0, s, p, n16, sink); break;
        default: return fail(KOEMI_ERR_INVALID, "stream read unroll must be 1, 2, 4 or 8");
    }
    return check_launch("koemi_stream_read");
}
