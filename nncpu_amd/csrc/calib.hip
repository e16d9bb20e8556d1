// Calibration kernels for the roofline denominators (libnncpu_calib.so,
// include/nncpu_calib.h): a read stream for the HBM rate at a given size and
// matrix-unit loops for the dense MFMA rates. Not part of the matmul path;
// the benchmark measures the box with them.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "nncpu_calib.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Each thread reads U 16-byte pieces (all issued before any is used) of a
// contiguous 16 * U * blockDim-byte span per workgroup, folds them with xor
// and writes one word per thread only if it is a value that never occurs
// (so the loads cannot be removed and nothing is written).
template <int U>
__global__ __launch_bounds__(256) void read_stream_kernel(const v4i* __restrict__ p, size_t n16, int* __restrict__ out) {
    const size_t base = ((size_t)blockIdx.x * U) * blockDim.x + threadIdx.x;
    v4i v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = base + (size_t)u * blockDim.x;
        v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : v4i{0, 0, 0, 0};
    }
    int acc = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x7F3A9C15) out[0] = acc;
}

// Four independent accumulator chains per wave, `iters` MFMAs each, so the
// matrix unit never waits on a result; the operands are lane values that the
// compiler cannot fold. A lane writes only if its sum is a value that never
// occurs.
__global__ __launch_bounds__(256) void mfma_i8_kernel(int iters, int* __restrict__ out) {
    const int a = (int)(threadIdx.x * 0x01010101u + 0x01020304u);
    const int b = (int)(threadIdx.x * 0x02030405u + 0x03010201u);
    const v4i A = {a, b, a ^ b, a + b}, B = {b, a, a + b, a ^ b};
    v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(B, A, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, A, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(B, B, c3, 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c0[r] ^ c1[r] ^ c2[r] ^ c3[r];
    if (s == 0x6B2D11F7) out[threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void mfma_bf16_kernel(int iters, int* __restrict__ out) {
    const float fa = 1.0f + threadIdx.x * 0.0078125f, fb = 2.0f - threadIdx.x * 0.00390625f;
    v8bf A, B;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        A[k] = (__bf16)(fa + k);
        B[k] = (__bf16)(fb - k);
    }
    v16f c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; ++i) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(B, A, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, A, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(B, B, c3, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
    if (s == 1234.5f) out[threadIdx.x] = 1;
}

// The shader clock under a light load: each workgroup's first lane reads
// the core-clock counter (s_memtime) and the constant 100 MHz counter
// (s_memrealtime) around a dependent FMA chain of `iters` steps, and stores
// the two differences (vector stores). cycles / (ticks / 100 MHz) is the
// clock the workgroup's CU ran at.
__global__ __launch_bounds__(64) void clock_probe_kernel(int iters, unsigned long long* __restrict__ out) {
    float v = 1.0f + threadIdx.x * 1e-7f;
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i) v = __builtin_fmaf(v, 0.999999f, 1e-7f);
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        out[2 * blockIdx.x] = c1 - c0;
        out[2 * blockIdx.x + 1] = (r1 - r0) + (v == 12345.0f ? 1 : 0);
    }
}

}  // namespace

extern "C" {

int nnc_clock_probe(int blocks, int iters, void* out, void* stream) {
    if (!out || blocks <= 0 || iters <= 0) return 1;
    clock_probe_kernel<<<blocks, 64, 0, (hipStream_t)stream>>>(iters, (unsigned long long*)out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}


int nnc_read_stream(const void* p, size_t bytes, int unroll, void* out, void* stream) {
    if (!p || !out || bytes % 16 != 0 || bytes == 0) return 1;
    const size_t n16 = bytes / 16;
    hipStream_t st = (hipStream_t)stream;
    if (unroll == 16) {
        const size_t wg = (n16 + 16 * 256 - 1) / (16 * 256);
        read_stream_kernel<16><<<(unsigned)wg, 256, 0, st>>>((const v4i*)p, n16, (int*)out);
    } else if (unroll == 4) {
        const size_t wg = (n16 + 4 * 256 - 1) / (4 * 256);
        read_stream_kernel<4><<<(unsigned)wg, 256, 0, st>>>((const v4i*)p, n16, (int*)out);
    } else {
        return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

long long nnc_mfma_ops(int kind, int iters, int blocks) {
    const long long per = kind == NNC_MFMA_I8 ? 2LL * 32 * 32 * 32 : 2LL * 32 * 32 * 16;
    return per * 4 * iters * (long long)blocks * 4;  // 4 chains, 4 waves per workgroup
}

int nnc_mfma_loop(int kind, int iters, int blocks, void* out, void* stream) {
    if (!out || iters <= 0 || blocks <= 0) return 1;
    hipStream_t st = (hipStream_t)stream;
    if (kind == NNC_MFMA_I8)
        mfma_i8_kernel<<<blocks, 256, 0, st>>>(iters, (int*)out);
    else if (kind == NNC_MFMA_BF16)
        mfma_bf16_kernel<<<blocks, 256, 0, st>>>(iters, (int*)out);
    else
        return 1;
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
