// Device forms of the CPU forward's scalar non-matmul arithmetic (gemma3.cpp,
// restating crates/nncpu/src/kernels/scalar.rs), shared by the decode step
// (gemma3_gpu.hip) and the layer kernels (layers_gpu.hip). Every function
// performs the CPU code's operations in its order, each rounded once
// (__f*_rn: the translation units are built with -ffp-contract=off too), so
// the results are the CPU restatement's bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>

#include "rmsnorm_exact.h"

namespace {

__device__ __forceinline__ float bf16f(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ uint16_t to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// scalar.rs:19-84 (gemma3.cpp exp_lane).
__device__ float exp_lane(float x) {
    const float EXP_LO = -87.336544f, EXP_HI = 88.722839f;
    const float LOG2E = 1.44269504088896340736f, LN2_HI = 0.693359375f, LN2_LO = -2.12194440e-4f;
    x = x > EXP_LO ? x : EXP_LO;
    x = x < EXP_HI ? x : EXP_HI;
    const float fx = __fsub_rn(__fadd_rn(__fmul_rn(x, LOG2E), 12582912.0f), 12582912.0f);
    float r = __fmaf_rn(-fx, LN2_HI, x);
    r = __fmaf_rn(-fx, LN2_LO, r);
    float y = __fmaf_rn(1.9875691500e-4f, r, 1.3981999507e-3f);
    y = __fmaf_rn(y, r, 8.3334519073e-3f);
    y = __fmaf_rn(y, r, 4.1665795894e-2f);
    y = __fmaf_rn(y, r, 1.6666665459e-1f);
    y = __fmaf_rn(y, r, 5.0000001201e-1f);
    y = __fmaf_rn(y, __fmul_rn(r, r), r);
    y = __fadd_rn(y, 1.0f);
    const float p2 = __uint_as_float((uint32_t)((int32_t)fx + 127) << 23);
    return __fmul_rn(y, p2);
}

// scalar.rs:86-103 (gemma3.cpp gelu_lane).
__device__ float gelu_lane(float v) {
    const float GELU_C = 0.79788456080286535f, GELU_A = 0.044715f;
    const float v3 = __fmul_rn(__fmul_rn(v, v), v);
    const float u = __fmul_rn(GELU_C, __fmaf_rn(GELU_A, v3, v));
    const float u2 = __fmul_rn(u, u), u4 = __fmul_rn(u2, u2), u6 = __fmul_rn(u4, u2);
    const float num = __fmul_rn(u, __fadd_rn(u6, __fmaf_rn(378.0f, u4, __fmaf_rn(17325.0f, u2, 135135.0f))));
    const float den = __fmaf_rn(28.0f, u6, __fmaf_rn(3150.0f, u4, __fmaf_rn(62370.0f, u2, 135135.0f)));
    const float t = fabsf(u) >= 5.0f ? copysignf(1.0f, u) : __fdiv_rn(num, den);
    return __fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, t));
}

// scalar.rs:104-106 (gemma3.cpp sigmoid_lane): 1 / (1 + exp(0 - g)), a true divide.
__device__ __forceinline__ float sigmoid_lane(float g) {
    return __fdiv_rn(1.0f, __fadd_rn(1.0f, exp_lane(__fsub_rn(0.0f, g))));
}

// (float)(1 / sqrt(ss / dim + eps)) in f64 (scalar.rs:232-292, gemma3.cpp
// rmsnorm_gamma_multi), ss the sum of squares as a double.
__device__ __forceinline__ float rms_of_d(double ss, int dim, float eps) { return nnh::rms_scale(ss, dim, eps); }
__device__ __forceinline__ float rms_of(float ss, int dim, float eps) { return rms_of_d((double)ss, dim, eps); }

}  // namespace

// ---- expf as glibc computes it ----------------------------------------------------------
// scalar.rs attn_merge (gemma3.cpp attn_merge) scales the partials by
// std::exp of a float: glibc's expf, the published algorithm of ARM's
// optimized-routines (glibc >= 2.28): z = x * 32 / ln2 in double, k = z
// rounded to an integer (by adding and subtracting 1.5 * 2^52), r = z - k,
// s = 2^(k / 32) from a 32-entry table of 2^(i / 32) with k's integer part
// added to the exponent, exp2(r / 32) by a degree-3 polynomial, one rounding
// to float. glibc's x86-64 FMA build contracts r = z - k into one fma of
// x * (32 / ln2) - k, so this does too. T[i] = bits of 2^(i / 32) rounded
// to double, minus i << 47 (expf_table). The CPU test runs every float
// through this and glibc's expf.
__host__ __device__ inline float glibc_expf(float x, const uint64_t* T) {
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42bu) {  // |x| >= 88
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double InvLn2N = 0x1.71547652b82fep+5, SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-20, C1 = 0x1.ebfce50fac4f3p-13, C2 = 0x1.62e42ff0c52d6p-6;
    const double xd = (double)x, z = InvLn2N * xd;
    double kd = z + SHIFT;
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= SHIFT;
    const double r = fma(InvLn2N, xd, -kd);
    const uint64_t t = T[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double zz = fma(C0, r, C1), r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(zz, r2, y);
    return (float)(y * s);
}

// The table of glibc_expf: bits of 2^(i / 32) rounded to double, minus i << 47.
inline void expf_table(uint64_t* T) {
    for (int i = 0; i < 32; ++i) {
        const double v = (double)exp2l((long double)i / 32);
        uint64_t u;
        memcpy(&u, &v, 8);
        T[i] = u - ((uint64_t)i << 47);
    }
}
