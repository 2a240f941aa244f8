// Shared device/host helpers for the gfx950 HERM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/koemi_hip.h"

namespace koemi {

// ----------------------------------------------------------------- errors ---
// Per-host-thread message for koemi_last_error(); set_error returns the status
// so entry points can `return fail(...)`.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

template <typename... Args>
inline int fail(int status, const char* fmt, Args... args) {
    set_error(fmt, args...);
    return status;
}
inline int fail(int status, const char* msg) {
    set_error("%s", msg);
    return status;
}

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return fail(KOEMI_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(err));
    }
    return KOEMI_OK;
}

inline hipStream_t as_stream(koemi_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------ element types ---
using bf16 = __bf16;
using f16 = _Float16;

template <typename T> struct AccOf { using type = float; };
template <> struct AccOf<double> { using type = double; };

template <typename T> __device__ __forceinline__ float to_f32(T v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }

// ------------------------------------------------------------ wave helpers ---
constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & (kWave - 1)); }

__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max_xor(float v) {
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    const int l = lane_id();
    return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// Exclusive prefix sum of one value per thread over a workgroup of THREADS
// threads (a multiple of 64): a wave-level shuffle scan, the wave totals
// scanned by every thread from LDS, two barriers. `wave_tot` is LDS scratch of
// THREADS / 64 entries. Also returns the workgroup total.
template <int THREADS, typename V>
__device__ __forceinline__ V block_exclusive_scan(V v, V* wave_tot, V& total) {
    const int lane = lane_id(), w = static_cast<int>(threadIdx.x) / kWave;
    V incl = v;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const V up = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += up;
    }
    if (lane == kWave - 1) wave_tot[w] = incl;
    __syncthreads();
    V before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < THREADS / kWave; ++i) {
        const V t = wave_tot[i];
        if (i < w) before += t;
        all += t;
    }
    __syncthreads();
    total = all;
    return before + incl - v;
}

// Number of blocks for `items` work items of `per_block` each, clamped to a grid size
// the runtime accepts.
// Gates of the bounded recurrent state (model/memory.py:22-26):
//   a = 2^-8 + (1 - 2^-7) sigmoid(zr),  b = (1 - a) tanh(zc).
// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32): absolute error below 1.5e-7 over all x.
// tanh(x) = 2 sigmoid(2x) - 1, the same two instructions: absolute error below
// 2.5e-7 over all x (tanh enters b, which adds to a state of order one, so the
// error is absolute; small arguments lose relative accuracy, not absolute);
// +-inf give +-1, NaN stays NaN.
__device__ __forceinline__ float gate_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}
__device__ __forceinline__ float gate_tanh(float x) {
    return fmaf(2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -2.88539008177792682f)), -1.0f);
}
constexpr float kGateMinRetention = 0.00390625f;        // 2^-8
constexpr float kGateRetentionSpan = 1.0f - 0.0078125f;  // (1 - 2^-8) - 2^-8 = 1 - 2^-7
// The working-state gates of one feature (model/memory.py:14-30 with the
// masking of network.py:307-309): retention a = 2^-8 + (1 - 2^-7) sigmoid(zr +
// br), candidate b = (1 - a) tanh(zc + bc); a masked position keeps the state
// (a = 1, b = 0).
__device__ __forceinline__ void gate_pair(float zr, float zc, float br, float bc, bool keep, float& a, float& b) {
    const float ga = kGateMinRetention + kGateRetentionSpan * gate_sigmoid(zr + br);
    const float gb = (1.0f - ga) * gate_tanh(zc + bc);
    a = keep ? ga : 1.0f;
    b = keep ? gb : 0.0f;
}

// Four consecutive values as fp32 (one 16-byte fp32 or 8-byte bf16 load).
// 16 bytes stored with a non-temporal hint: outputs written once and far
// larger than the caches (above KOEMI_NT_STORE_BYTES) skip them.
#ifndef KOEMI_NT_STORE_BYTES
#define KOEMI_NT_STORE_BYTES (int64_t(16) << 20)
#endif
__device__ __forceinline__ void store16_nt(void* p, const uint4& v) {
    typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
    const u32x4_nt w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4_nt*>(p));
}

__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const bf16* p) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
}
// Four consecutive outputs (one 16-byte fp32 or 8-byte bf16 store).
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
    const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<bf16>(a)) |
                        (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<bf16>(b))) << 16);
    const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<bf16>(c)) |
                        (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<bf16>(d))) << 16);
    *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

inline unsigned grid_for(int64_t items, int64_t per_block) {
    int64_t b = (items + per_block - 1) / per_block;
    if (b < 1) b = 1;
    return static_cast<unsigned>(b);
}

inline bool float_dtype(int dt) { return dt == KOEMI_F32 || dt == KOEMI_F16 || dt == KOEMI_BF16; }
inline bool index_dtype(int dt) { return dt == KOEMI_I32 || dt == KOEMI_I64; }
inline const char* dtype_name(int dt) {
    switch (dt) {
        case KOEMI_F32: return "float32";
        case KOEMI_F16: return "float16";
        case KOEMI_BF16: return "bfloat16";
        case KOEMI_F64: return "float64";
        case KOEMI_I32: return "int32";
        case KOEMI_I64: return "int64";
        case KOEMI_BOOL: return "bool";
        default: return "unknown";
    }
}

}  // namespace koemi
