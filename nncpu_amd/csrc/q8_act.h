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

}  // namespace nnh
