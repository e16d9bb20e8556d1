// nncpu's Q8_0 activation encoder (crates/nncpu/src/kernels/quant.rs:31-60),
// per value and per block of 32, for every device kernel that quantizes
// activations: the library's quantizer and the device forward's producer
// kernels that write a matmul's int8 input directly. One definition, so
// both give the same bits.
#pragma once

#include "common.h"

namespace nnh {

// Round half to even, then Rust's saturating `as i32` (quant.rs:18-29).
__device__ __forceinline__ int rint_sat(float v) {
    float r = __builtin_rintf(v);
    if (!(r == r)) return 0;
    if (r >= 2147483648.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int)0x80000000;
    return (int)r;
}

// |v| for the block maximum (quant.rs:43-48): NaNs are skipped (`v.abs() >
// amax` is false for them), so they count as 0; max is order-free over the rest.
__device__ __forceinline__ float q8_abs(float v) {
    const float a = fabsf(v);
    return a == a ? a : 0.0f;
}

// The block's BF16 scale from its maximum (amax times the reciprocal of 127,
// rounded to BF16, quant.rs:53-55) and the reciprocal the values are
// multiplied by (0 for an all-zero block).
struct Q8Scale {
    uint32_t bits;
    float scale, inv;
};
__device__ __forceinline__ Q8Scale q8_scale(float amax) {
    Q8Scale s;
    s.bits = f32_to_bf16(__fmul_rn(amax, 1.0f / 127.0f));
    s.scale = bf16f(s.bits);
    s.inv = s.scale > 0.0f ? __fdiv_rn(1.0f, s.scale) : 0.0f;
    return s;
}

// One value's quant, clamped to the symmetric range (quant.rs:56-58).
__device__ __forceinline__ int q8_quant(float v, float inv) {
    const int q = rint_sat(__fmul_rn(v, inv));
    return q < -127 ? -127 : (q > 127 ? 127 : q);
}

// Lane exchanges by DPP (a VALU operand modifier, no LDS round trip): 0xB1
// quad_perm [1,0,3,2], 0x4E quad_perm [2,3,0,1], 0x141 row_half_mirror (lane
// i <-> 7 - i within 8), 0x140 row_mirror (i <-> 15 - i within 16). After
// the first k of them every lane holds the max / sum over its aligned group
// of 2, 4, 8, 16 lanes (max and integer sums do not depend on the order).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float max8(float a) {
    a = fmaxf(a, dpp_f<0xB1>(a));
    a = fmaxf(a, dpp_f<0x4E>(a));
    return fmaxf(a, dpp_f<0x141>(a));
}
__device__ __forceinline__ int sum8(int a) {
    a += dpp_i<0xB1>(a);
    a += dpp_i<0x4E>(a);
    return a + dpp_i<0x141>(a);
}

// A thread's pieces k = 0 .. K-1 of a row, piece k being values 4i .. 4i+3
// with i = i0 + k * stride (i0 & 7 == lane & 7, stride a multiple of 8), so
// a block is one piece of each of 8 consecutive lanes. Every lane of the
// wave calls it, pieces at i >= n4 holding zeros (a whole block is in range
// or not); each step runs over all pieces before the next, so the pieces'
// chains overlap. For each piece in range, put(i, word, scale, qsum): the
// four quants as one little-endian word, the block's scale and the sum of
// its quants (the same in all 8 lanes of the block).
template <int K, class Put>
__device__ __forceinline__ void q8_pieces(const float4 (&p)[K], int i0, int stride, int n4, Put&& put) {
    float a[K];
    Q8Scale s[K];
    int q[K][4], qs[K];
#pragma unroll
    for (int k = 0; k < K; ++k)
        a[k] = max8(fmaxf(fmaxf(q8_abs(p[k].x), q8_abs(p[k].y)), fmaxf(q8_abs(p[k].z), q8_abs(p[k].w))));
#pragma unroll
    for (int k = 0; k < K; ++k) {
        s[k] = q8_scale(a[k]);
        q[k][0] = q8_quant(p[k].x, s[k].inv);
        q[k][1] = q8_quant(p[k].y, s[k].inv);
        q[k][2] = q8_quant(p[k].z, s[k].inv);
        q[k][3] = q8_quant(p[k].w, s[k].inv);
        qs[k] = sum8(q[k][0] + q[k][1] + q[k][2] + q[k][3]);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = i0 + k * stride;
        if (i >= n4) continue;
        put(i,
            (uint32_t)(q[k][0] & 255) | (uint32_t)(q[k][1] & 255) << 8 | (uint32_t)(q[k][2] & 255) << 16 |
                (uint32_t)(q[k][3] & 255) << 24,
            s[k], qs[k]);
    }
}

}  // namespace nnh
