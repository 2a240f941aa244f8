// rocBLAS handles for the plain GEMMs of the salient read and the recurrent
// gates: one per device, created on first use and kept for the process. The
// rocBLAS library is the one PyTorch has loaded (same HIP runtime). A handle
// carries its stream, so callers hold g_blas_mutex from setting the stream to
// the last call that uses it.
#include "common.hpp"

#include <rocblas/rocblas.h>

#include <mutex>

namespace koemi {

std::mutex g_blas_mutex;

namespace {
rocblas_handle g_blas[64] = {};
}  // namespace

rocblas_handle blas_handle(int device) {
    if (device < 0 || device >= 64) return nullptr;
    if (!g_blas[device] && rocblas_create_handle(&g_blas[device]) != rocblas_status_success) g_blas[device] = nullptr;
    return g_blas[device];
}

}  // namespace koemi
