// argmax over the lm_head logits with the reference's tie and NaN rules
// (crates/nncpu/src/model/forward.rs:1003-1011): the first largest value
// wins, a NaN never replaces the running best, and a NaN in row 0 keeps
// row 0 (every `v[i] > NaN` is false). Mode 1 is the BF16 4-row kernel's
// running best (kernels/scalar.rs:612-628): it starts from -inf with no row,
// so NaN and -inf are never taken and nothing taken gives row 0.
//
// Each candidate is one u64 key: an order-preserving image of the value in
// the high word (-0 folded onto +0, which compare equal), the complement of
// the index in the low word, so the integer maximum is the largest value at
// its lowest index. NaNs get key 0.

#include "common.h"

namespace nnh {
namespace {

constexpr int PER_BLOCK = 2048;

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ uint64_t block_max(uint64_t k) {
    __shared__ uint64_t part[4];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)k, m, 64);
        uint32_t hi = __shfl_xor((uint32_t)(k >> 32), m, 64);
        k = umax64(k, ((uint64_t)hi << 32) | lo);
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
    __syncthreads();
    return umax64(umax64(part[0], part[1]), umax64(part[2], part[3]));
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ v, size_t n,
                                                             uint64_t* __restrict__ partial) {
    size_t base = (size_t)blockIdx.x * PER_BLOCK;
    uint64_t k = 0;
    for (int i = threadIdx.x; i < PER_BLOCK; i += 256) {
        size_t e = base + i;
        if (e < n) k = umax64(k, argmax_key(v[e], (uint32_t)e));
    }
    k = block_max(k);
    if (threadIdx.x == 0) partial[blockIdx.x] = k;
}

// The key of -inf's high word: the largest key no value is taken with in mode 1.
constexpr uint32_t NEG_INF_KEY = ~0xff800000u;

__global__ __launch_bounds__(256) void argmax_final_kernel(const float* __restrict__ v, const uint64_t* __restrict__ partial,
                                                           int nparts, uint64_t* __restrict__ out, int mode) {
    uint64_t k = 0;
    for (int i = threadIdx.x; i < nparts; i += 256) k = umax64(k, partial[i]);
    k = block_max(k);
    if (threadIdx.x == 0) {
        float v0 = v[0];
        const bool none = mode == 1 ? (uint32_t)(k >> 32) <= NEG_INF_KEY : (k == 0 || !(v0 == v0));
        out[0] = none ? 0 : (uint64_t)(0xffffffffu - (uint32_t)k);
    }
}

}  // namespace

// Compute units of the current device (cached per device).
int cu_count() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

size_t argmax_partial_words(size_t n) { return (n + PER_BLOCK - 1) / PER_BLOCK; }

void launch_argmax_final(const float* v, const uint64_t* partial, int nparts, uint64_t* out, hipStream_t st,
                         int mode) {
    argmax_final_kernel<<<1, 256, 0, st>>>(v, partial, nparts, out, mode);
}

void launch_argmax(const float* v, size_t n, uint64_t* partial, uint64_t* out, hipStream_t st, int mode) {
    int nparts = (int)argmax_partial_words(n);
    argmax_partial_kernel<<<nparts, 256, 0, st>>>(v, n, partial);
    argmax_final_kernel<<<1, 256, 0, st>>>(v, partial, nparts, out, mode);
}

}  // namespace nnh
