// nncpu's RMSNorm scale, exactly: the sum of squares in scalar.rs's order
// (sum_sq, kernels/scalar.rs:232-250: eight FMA lanes, lane l over elements
// l, l + 8, ... of the whole 8-chunks, hsum8, then the tail in f64) and
// (float)(1 / sqrt(ss / dim + eps)) in f64 (scalar.rs:232-292). Shared by
// the library's fused norm-and-matmul kernels and the device forward.
#pragma once
#include <hip/hip_runtime.h>

namespace nnh {

// hsum8 of lanes 0..7's values (valid at lane 0 of each aligned group of 8):
// xor-4 gives v_l + v_{l+4}, xor-1 and xor-2 then add those pairs as hsum8 does.
__device__ __forceinline__ float rms_hsum8_lanes(float a) {
    const float p = __fadd_rn(a, __shfl_xor(a, 4, 64));
    const float q = __fadd_rn(p, __shfl_xor(p, 1, 64));
    return __fadd_rn(q, __shfl_xor(q, 2, 64));
}

// sum_sq of v[0..dim) (LDS), run by one wave: lanes 0..7 each run FMA lane l
// over the whole 8-chunks in order, hsum8, then the tail in f64. The result
// (a double) is returned to every lane. B: values per read batch (2 B
// registers; kernels that must stay lean pass a smaller one).
template <int B = 32>
__device__ __forceinline__ double rms_sumsq(const float* v, int dim, int lane) {
    const int body = dim & ~7;
    float a = 0.0f;
    if (lane < 8) {
        // The lane's values B at a time, each batch read while the previous
        // batch's FMAs run (the chain itself is sequential); two named
        // buffers in turn, so no register array is indexed at run time.
        int i = lane;
        float ta[B], tb[B];
        auto full = [&](int at) { return at + 8 * (B - 1) < body; };
        if (full(i)) {
#pragma unroll
            for (int k = 0; k < B; ++k) ta[k] = v[i + 8 * k];
            while (true) {
                const bool nb = full(i + 8 * B);
                if (nb) {
#pragma unroll
                    for (int k = 0; k < B; ++k) tb[k] = v[i + 8 * B + 8 * k];
                }
#pragma unroll
                for (int k = 0; k < B; ++k) a = __fmaf_rn(ta[k], ta[k], a);
                i += 8 * B;
                if (!nb) break;
                const bool na = full(i + 8 * B);
                if (na) {
#pragma unroll
                    for (int k = 0; k < B; ++k) ta[k] = v[i + 8 * B + 8 * k];
                }
#pragma unroll
                for (int k = 0; k < B; ++k) a = __fmaf_rn(tb[k], tb[k], a);
                i += 8 * B;
                if (!na) break;
            }
        }
        for (; i < body; i += 8) a = __fmaf_rn(v[i], v[i], a);
    }
    const float h = rms_hsum8_lanes(a);
    double s = dim >= 8 ? (double)__shfl(h, 0, 64) : 0.0;
    for (int i = body; i < dim; ++i) s = __dadd_rn(s, __dmul_rn((double)v[i], (double)v[i]));
    return s;
}

// The same sum of squares from a chain-major copy: FMA lane l's values
// (elements l, l + 8, ...) contiguous at vt + l * stride (rms_t_stride),
// read 16 bytes at a time, B of those per batch, the next batch's reads in
// flight while the current batch's FMAs run. dim a multiple of 32 (no tail).
// Run by one wave; the result is returned to every lane.
__host__ __device__ inline int rms_t_stride(int dim) { return dim / 8 + 4; }  // 16-byte rows, staggered banks
template <int B = 8>
__device__ __forceinline__ double rms_sumsq_t(const float* vt, int dim, int lane) {
    const int nq = dim / 32;  // 16-byte reads per FMA lane
    const int nfull = nq / B;
    float a = 0.0f;
    if (lane < 8) {
        const float4* p = (const float4*)(vt + lane * rms_t_stride(dim));
        float4 ta[B], tb[B];
        auto fma4 = [&](const float4& v) {
            a = __fmaf_rn(v.x, v.x, a);
            a = __fmaf_rn(v.y, v.y, a);
            a = __fmaf_rn(v.z, v.z, a);
            a = __fmaf_rn(v.w, v.w, a);
        };
        if (nfull > 0) {
#pragma unroll
            for (int k = 0; k < B; ++k) ta[k] = p[k];
            // Batch reads are clamped to the last whole batch (rereads past
            // the end are never used), so the loop has no divergent loads.
            // The scheduling barriers keep each batch's reads ahead of the
            // previous batch's FMAs (the compiler would sink them).
            for (int t = 0;; t += 2) {
                const float4* q1 = p + B * min(t + 1, nfull - 1);
#pragma unroll
                for (int k = 0; k < B; ++k) tb[k] = q1[k];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int k = 0; k < B; ++k) fma4(ta[k]);
                if (t + 1 >= nfull) break;
                const float4* q2 = p + B * min(t + 2, nfull - 1);
#pragma unroll
                for (int k = 0; k < B; ++k) ta[k] = q2[k];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int k = 0; k < B; ++k) fma4(tb[k]);
                if (t + 2 >= nfull) break;
            }
        }
        for (int k = B * nfull; k < nq; ++k) fma4(p[k]);
    }
    const float h = rms_hsum8_lanes(a);
    return (double)__shfl(h, 0, 64);
}

// (float)(1 / sqrt(ss / dim + eps)) with ss a double, in f64.
__device__ __forceinline__ float rms_scale(double ss, int dim, float eps) {
    const float inv_dim = __fdiv_rn(1.0f, (float)dim);
    return (float)__ddiv_rn(1.0, __dsqrt_rn(__dadd_rn(__dmul_rn(ss, (double)inv_dim), (double)eps)));
}

}  // namespace nnh
