// Load-time re-encoding on the device: nncpu's f32 -> Q8_0 and f32 -> Q4
// encoders (crates/nncpu/src/kernels/quant.rs:31-95), bit for bit, one
// 32-lane half-wave per block of 32 values.
//
// The reference walks a block sequentially: Q8_0 takes amax with
// `v.abs() > amax` from 0 (NaNs never win); Q4 takes lo / hi from b[0] with
// strict `v < lo` / `v > hi`, so among equal candidates (e.g. -0.0 and 0.0)
// the first in the block wins, and a NaN in b[0] leaves lo = hi = NaN. The
// lane reductions here carry the block index with the value to reproduce
// exactly that.

#include "common.h"

namespace nnh {
namespace {

__device__ __forceinline__ int rint_sat_enc(float v) {
    float r = __builtin_rintf(v);
    if (!(r == r)) return 0;
    if (r >= 2147483648.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int)0x80000000;
    return (int)r;
}

// Q8_0: qs[n], scales[n/32] (quant.rs:31-60).
__global__ __launch_bounds__(256) void encode_q8_kernel(const float* __restrict__ w, size_t nblocks,
                                                        int8_t* __restrict__ qs, uint16_t* __restrict__ sc) {
    const int k = threadIdx.x & 31;
    const size_t blk = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const bool valid = blk < nblocks;
    const size_t b = valid ? blk : 0;
    const float v = w[32 * b + k];
    float a = fabsf(v);
    a = (a == a) ? a : 0.0f;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m, 32));
    const uint32_t sbits = f32_to_bf16(__fmul_rn(a, 1.0f / 127.0f));
    const float scale = bf16f(sbits);
    const float inv = scale > 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
    int q = rint_sat_enc(__fmul_rn(v, inv));
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    if (!valid) return;
    qs[32 * b + k] = (int8_t)q;
    if (k == 0) sc[b] = (uint16_t)sbits;
}

// Q4: qs[n/2], scales[n/32], biases[n/32] (quant.rs:62-95).
__global__ __launch_bounds__(256) void encode_q4_kernel(const float* __restrict__ w, size_t nblocks,
                                                        uint8_t* __restrict__ qs, uint16_t* __restrict__ sc,
                                                        uint16_t* __restrict__ bi) {
    const int k = threadIdx.x & 31;
    const size_t blk = (size_t)blockIdx.x * 8 + (threadIdx.x >> 5);
    const bool valid = blk < nblocks;
    const size_t b = valid ? blk : 0;
    const float v = w[32 * b + k];
    const float v0 = __shfl(v, 0, 32);
    float lo, hi;
    if (!(v0 == v0)) {
        lo = hi = v0;  // b[0] is NaN: nothing compares below or above it
    } else {
        // Over the non-NaN values (a NaN never replaces the running value):
        // min and max, the first occurrence among equal values.
        float lv = (v == v) ? v : v0, hv = lv;
        int li = (v == v) ? k : 0, hi_i = li;
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) {
            const float olv = __shfl_xor(lv, m, 32), ohv = __shfl_xor(hv, m, 32);
            const int oli = __shfl_xor(li, m, 32), ohi = __shfl_xor(hi_i, m, 32);
            if (olv < lv || (olv == lv && oli < li)) lv = olv, li = oli;
            if (ohv > hv || (ohv == hv && ohi < hi_i)) hv = ohv, hi_i = ohi;
        }
        lo = lv;
        hi = hv;
    }
    const uint32_t sbits = f32_to_bf16(__fmul_rn(__fsub_rn(hi, lo), 1.0f / 15.0f));
    const uint32_t bbits = f32_to_bf16(lo);
    const float scale = bf16f(sbits), bias = bf16f(bbits);
    const float inv = scale > 0.0f ? __fdiv_rn(1.0f, scale) : 0.0f;
    int q = rint_sat_enc(__fmul_rn(__fsub_rn(v, bias), inv));
    q = q < 0 ? 0 : (q > 15 ? 15 : q);
    const int q_hi = __shfl_down(q, 16, 32);  // element k + 16 for lanes k < 16
    if (!valid) return;
    if (k < 16) qs[16 * b + k] = (uint8_t)(q | (q_hi << 4));
    if (k == 0) {
        sc[b] = (uint16_t)sbits;
        bi[b] = (uint16_t)bbits;
    }
}

}  // namespace

void launch_encode(int dtype, const float* w, size_t n, uint8_t* qs, uint16_t* sc, uint16_t* bi, hipStream_t st) {
    const size_t nblocks = n / 32;
    const int grid = (int)((nblocks + 7) / 8);
    if (dtype == 1)
        encode_q8_kernel<<<grid, 256, 0, st>>>(w, nblocks, (int8_t*)qs, sc);
    else
        encode_q4_kernel<<<grid, 256, 0, st>>>(w, nblocks, qs, sc, bi);
}

}  // namespace nnh
