// Reproducible fp32 exp and log for the kernels whose outputs are compared bit
// for bit (surprise scores feeding the admission mask, learned-router
// probabilities feeding top-k).
//
// Both routines use textbook methods with every rounding step spelled out
// (explicit fmaf, floating-point contraction disabled), so a scalar C
// evaluation that follows the same steps returns identical bits:
//
//   exp: Cody & Waite (1980) argument reduction x = n ln2 + r with ln2 split
//        into a 15-significant-bit head (n * head is exact for |n| < 256) and a
//        tail; e^r on |r| <= ln2/2 by a degree-6 polynomial in Horner form whose
//        coefficients were fitted for minimax relative error with each one
//        rounded to fp32 in turn, highest degree first (c0 = c1 = 1; relative
//        error 3.8e-9 with the fp32 coefficients, below the degree-7 Taylor
//        polynomial's); the result is scaled by 2^n with ldexp, exact because
//        inputs below -86 return 0 (the scaled result is never subnormal).
//        Inputs above 88 return +inf.
//   log: x = m 2^e with m in [sqrt(1/2), sqrt(2)); log m = 2 atanh(f),
//        f = (m - 1) / (m + 1), by the odd series 2 (f + f^3/3 + ... + f^9/9)
//        (|f| <= 0.1716, truncation < 3e-9 relative); log x = e ln2 + log m.
#pragma once

#include <cstdint>

namespace koemi {
namespace detmath {

constexpr float kLog2e = 1.4426950216293335f;
constexpr float kLn2Hi = 0.693145751953125f;       // 0x3f317200
constexpr float kLn2Lo = 1.428606765330187e-06f;   // ln2 - kLn2Hi
constexpr float kSqrt2 = 1.4142135381698608f;

__host__ __device__ __forceinline__ float bits_to_float(uint32_t u) {
    union { uint32_t u; float f; } c;
    c.u = u;
    return c.f;
}
__host__ __device__ __forceinline__ uint32_t float_to_bits(float f) {
    union { uint32_t u; float f; } c;
    c.f = f;
    return c.u;
}

// Coefficients c6 .. c2 of the exp polynomial (bit patterns 0x3ab51225,
// 0x3c091cea, 0x3d2aac79, 0x3e2aaa49, 0x3efffffe).
constexpr float kExpC6 = 0.0013814611593261361f;
constexpr float kExpC5 = 0.008368710055947304f;
constexpr float kExpC4 = 0.04166838899254799f;
constexpr float kExpC3 = 0.1666652113199234f;
constexpr float kExpC2 = 0.4999999403953552f;

// e^x for -86 <= x <= 88 (the reduction and polynomial of det_expf); a NaN
// input gives a NaN.
__device__ __forceinline__ float det_exp_core(float x) {
#pragma clang fp contract(off)
    const float n = __builtin_rintf(x * kLog2e);
    float r = __builtin_fmaf(-n, kLn2Hi, x);
    r = __builtin_fmaf(-n, kLn2Lo, r);
    float p = kExpC6;
    p = __builtin_fmaf(p, r, kExpC5);
    p = __builtin_fmaf(p, r, kExpC4);
    p = __builtin_fmaf(p, r, kExpC3);
    p = __builtin_fmaf(p, r, kExpC2);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_amdgcn_ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float det_expf(float x) {
    if (x != x) return x;
    if (x < -86.0f) return 0.0f;
    if (x > 88.0f) return __builtin_inff();
    return det_exp_core(x);
}

// det_expf for arguments known not to exceed 0 (x - max(x) terms of a
// softmax, or NaN): the same bits without the overflow test; a NaN input
// propagates through the arithmetic (a NaN out, payload unspecified).
__device__ __forceinline__ float det_expf_nonpos(float x) {
    const float e = det_exp_core(x);
    return x < -86.0f ? 0.0f : e;
}

__device__ __forceinline__ float det_logf(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    int e_adj = 0;
    if (x < 1.1754943508222875e-38f) {  // subnormal: rescale by 2^24
        x = x * 16777216.0f;
        e_adj = -24;
    }
    const uint32_t u = float_to_bits(x);
    int e = static_cast<int>((u >> 23) & 0xffu) - 127 + e_adj;
    float m = bits_to_float((u & 0x007fffffu) | 0x3f800000u);
    if (m > kSqrt2) {
        m = m * 0.5f;
        e += 1;
    }
    const float f = (m - 1.0f) / (m + 1.0f);
    const float s = f * f;
    float p = 1.111111119389534e-01f;                 // 1/9
    p = __builtin_fmaf(p, s, 1.428571492433548e-01f);  // 1/7
    p = __builtin_fmaf(p, s, 2.0000000298023224e-01f); // 1/5
    p = __builtin_fmaf(p, s, 3.333333432674408e-01f);  // 1/3
    const float fs = f * s;
    const float atanh_f = __builtin_fmaf(fs, p, f);
    const float log_m = atanh_f * 2.0f;
    const float ef = static_cast<float>(e);
    return __builtin_fmaf(ef, kLn2Hi, __builtin_fmaf(ef, kLn2Lo, log_m));
}

}  // namespace detmath
}  // namespace koemi
