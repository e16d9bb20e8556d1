// Load-time decoding of GGUF tensor blocks to f32 on the device
// (crates/nncpu/src/kernels/quant.rs:97-291, dequantize_to_f32), the step
// model/load.rs:182-206 runs before re-encoding a matrix to nncpu's layouts:
// F32 (0), F16 (1), BF16 (30), Q4_0 (2), Q4_1 (3), Q5_0 (6), Q5_1 (7),
// Q8_0 (8), Q4_K (12), Q5_K (13), Q6_K (14). Every value is the reference's
// bit for bit: the fp16 conversion is done on the bits as runtime.rs:25-48
// does it (subnormals renormalised, NaN payloads kept), and the products and
// sums are separate f32 operations in the reference's order
// (-ffp-contract=off). One thread per 32 outputs (a classic block, or a
// sub-block run of a 256-value K-quant block); per value for the float types.

#include "common.h"

namespace nnh {
namespace {

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            // Subnormal: shift the mantissa up to its leading one.
            const int lz = __builtin_clz(mant) - 21;  // leading zeros within the 11-bit field
            const uint32_t m = mant << lz;
            bits = sign | ((uint32_t)(127 - 15 + 1 - lz) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return __uint_as_float(bits);
}

__device__ __forceinline__ float f16_at(const uint8_t* b, int i) {
    return f16_bits_to_f32((uint32_t)b[i] | ((uint32_t)b[i + 1] << 8));
}

// quant.rs:163-195: one classic block per thread.
template <bool HAS_MIN, bool HAS_HIGH>
__global__ void dequant_legacy_kernel(const uint8_t* __restrict__ src, size_t nblocks, float* __restrict__ dst) {
    constexpr int BYTES = 2 + (HAS_MIN ? 2 : 0) + (HAS_HIGH ? 4 : 0) + 16;
    constexpr int CENTRE = HAS_MIN ? 0 : HAS_HIGH ? 16 : 8;
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const uint8_t* p = src + bi * BYTES;
    float* y = dst + 32 * bi;
    const float d = f16_at(p, 0), m = HAS_MIN ? f16_at(p, 2) : 0.0f;
    constexpr int O = HAS_MIN ? 4 : 2;
    const uint32_t qh = HAS_HIGH ? (uint32_t)p[O] | (uint32_t)p[O + 1] << 8 | (uint32_t)p[O + 2] << 16 |
                                       (uint32_t)p[O + 3] << 24
                                 : 0u;
    const uint8_t* qs = p + BYTES - 16;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int hi0 = (int)(((qh >> j) << 4) & 0x10u), hi1 = (int)((qh >> (j + 12)) & 0x10u);
        y[j] = __fadd_rn(__fmul_rn((float)(((int)(qs[j] & 0x0f) | hi0) - CENTRE), d), m);
        y[j + 16] = __fadd_rn(__fmul_rn((float)(((int)(qs[j] >> 4) | hi1) - CENTRE), d), m);
    }
}

// block_q8_0 = { fp16 d; int8 qs[32] } (quant.rs:141-149).
__global__ void dequant_q8_0_kernel(const uint8_t* __restrict__ src, size_t nblocks, float* __restrict__ dst) {
    const size_t bi = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    const uint8_t* b = src + 34 * bi;
    const float d = f16_at(b, 0);
#pragma unroll
    for (int k = 0; k < 32; ++k) dst[32 * bi + k] = __fmul_rn(d, (float)(int8_t)b[2 + k]);
}

// quant.rs:197-211.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, float& d, float& m) {
    uint32_t dd, mm;
    if (j < 4) {
        dd = q[j] & 63u;
        mm = q[j + 4] & 63u;
    } else {
        dd = (q[j + 4] & 0x0fu) | ((uint32_t)(q[j - 4] >> 6) << 4);
        mm = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
    }
    d = (float)dd;
    m = (float)mm;
}

// quant.rs:213-266: thread t of a block makes outputs 32t..32t+32 (run t/2,
// the low nibbles for even t, the high for odd).
template <bool Q5>
__global__ void dequant_qk_kernel(const uint8_t* __restrict__ src, size_t nblocks, float* __restrict__ dst) {
    constexpr int BYTES = Q5 ? 176 : 144;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks * 8) return;
    const size_t bi = i / 8;
    const int t = (int)(i % 8), j = t / 2, hi = t & 1;
    const uint8_t* b = src + bi * BYTES;
    const float d = f16_at(b, 0), dmin = f16_at(b, 2);
    float sc, mn;
    scale_min_k4(2 * j + hi, b + 4, sc, mn);
    const float d1 = __fmul_rn(d, sc), m1 = __fmul_rn(dmin, mn);
    const uint8_t* q = b + (Q5 ? 48 : 16) + 32 * j;
    const uint8_t* qh = b + 16;
    const uint32_t u = 1u << (2 * j + hi);
    float* y = dst + bi * 256 + 64 * j + 32 * hi;
#pragma unroll 8
    for (int l = 0; l < 32; ++l) {
        const uint32_t nib = hi ? (uint32_t)(q[l] >> 4) : (uint32_t)(q[l] & 0x0f);
        const uint32_t h = Q5 && (qh[l] & u) ? 16u : 0u;
        y[l] = __fsub_rn(__fmul_rn(d1, (float)(nib + h)), m1);
    }
}

// quant.rs:268-291: thread t of a block makes half t/4's outputs
// 32 (t%4) .. +32 of that half.
__global__ void dequant_q6k_kernel(const uint8_t* __restrict__ src, size_t nblocks, float* __restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks * 8) return;
    const size_t bi = i / 8;
    const int t = (int)(i % 8), h = t / 4, part = t % 4;
    const uint8_t* b = src + bi * 210;
    const float d = f16_at(b, 208);
    const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
    const int8_t* sc = (const int8_t*)(b + 192 + 8 * h);
    float* y = dst + bi * 256 + 128 * h + 32 * part;
#pragma unroll 8
    for (int l = 0; l < 32; ++l) {
        const int is = l / 16;
        int q;
        if (part == 0)
            q = (int)((ql[l] & 0x0f) | ((qh[l] & 3) << 4)) - 32;
        else if (part == 1)
            q = (int)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
        else if (part == 2)
            q = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        else
            q = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        y[l] = __fmul_rn(__fmul_rn(d, (float)sc[is + 2 * part]), (float)q);
    }
}

// F32 (bits as they are), F16 and BF16, one value per thread.
__global__ void dequant_float_kernel(uint32_t type, const uint8_t* __restrict__ src, size_t n, float* __restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (type == 0) {
        const uint32_t v = (uint32_t)src[4 * i] | (uint32_t)src[4 * i + 1] << 8 | (uint32_t)src[4 * i + 2] << 16 |
                           (uint32_t)src[4 * i + 3] << 24;
        dst[i] = __uint_as_float(v);
    } else {
        const uint32_t v = (uint32_t)src[2 * i] | (uint32_t)src[2 * i + 1] << 8;
        dst[i] = type == 1 ? f16_bits_to_f32(v) : bf16f(v);
    }
}

inline unsigned blocks_for(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

bool ggml_block(uint32_t t, size_t* bytes, size_t* per) {
    switch (t) {
        case 0: *bytes = 4, *per = 1; return true;
        case 1: case 30: *bytes = 2, *per = 1; return true;
        case 2: *bytes = 18, *per = 32; return true;
        case 3: *bytes = 20, *per = 32; return true;
        case 6: *bytes = 22, *per = 32; return true;
        case 7: *bytes = 24, *per = 32; return true;
        case 8: *bytes = 34, *per = 32; return true;
        case 12: *bytes = 144, *per = 256; return true;
        case 13: *bytes = 176, *per = 256; return true;
        case 14: *bytes = 210, *per = 256; return true;
        default: return false;
    }
}

void launch_dequantize(uint32_t t, const uint8_t* src, size_t n, float* dst, hipStream_t st) {
    size_t bytes, per;
    if (!ggml_block(t, &bytes, &per) || n == 0) return;
    const size_t nb = n / per;
    switch (t) {
        case 0: case 1: case 30: dequant_float_kernel<<<blocks_for(n), 256, 0, st>>>(t, src, n, dst); break;
        case 2: dequant_legacy_kernel<false, false><<<blocks_for(nb), 256, 0, st>>>(src, nb, dst); break;
        case 3: dequant_legacy_kernel<true, false><<<blocks_for(nb), 256, 0, st>>>(src, nb, dst); break;
        case 6: dequant_legacy_kernel<false, true><<<blocks_for(nb), 256, 0, st>>>(src, nb, dst); break;
        case 7: dequant_legacy_kernel<true, true><<<blocks_for(nb), 256, 0, st>>>(src, nb, dst); break;
        case 8: dequant_q8_0_kernel<<<blocks_for(nb), 256, 0, st>>>(src, nb, dst); break;
        case 12: dequant_qk_kernel<false><<<blocks_for(nb * 8), 256, 0, st>>>(src, nb, dst); break;
        case 13: dequant_qk_kernel<true><<<blocks_for(nb * 8), 256, 0, st>>>(src, nb, dst); break;
        case 14: dequant_q6k_kernel<<<blocks_for(nb * 8), 256, 0, st>>>(src, nb, dst); break;
        default: break;
    }
}

}  // namespace nnh
