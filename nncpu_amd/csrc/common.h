// Shared device helpers and launcher declarations for libnncpu_hip.so.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace nnh {

// BF16 bits -> f32, exact (the BF16 bits are the high half of the f32;
// crates/nncpu/src/runtime.rs:10-13).
__device__ __forceinline__ float bf16f(uint32_t v) { return __uint_as_float(v << 16); }

// f32 -> BF16 bits, round to nearest even (runtime.rs:15-21).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Lane-exchange sums used by the reduction trees. `__shfl_xor` moves data
// through the LDS crossbar without touching LDS memory.
__device__ __forceinline__ float xor_get(float v, int mask) { return __shfl_xor(v, mask, 64); }
__device__ __forceinline__ double xor_get(double v, int mask) { return __shfl_xor(v, mask, 64); }

inline int ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// ---- launchers (defined beside their kernels) -------------------------------

// Upload-time relayouts for the bit-exact f32 path (kernels_f32.hip).
void launch_relayout_f32(int dtype, const uint8_t* raw_qs, const uint16_t* raw_scales, uint8_t* fq, uint16_t* fs,
                         int rows, int nb, int nbp, hipStream_t st);
// Q4 block sums of n_tok vectors (kernels/scalar.rs:355-359 tree).
void launch_block_sums(const float* x, size_t x_stride, int nb, int n_tok, float* xsum, hipStream_t st);
// Bit-exact f32 gemv for n_tok <= 16 vectors.
void launch_gemv_f32(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases, const float* x,
                     size_t x_stride, const float* xsum, int rows, int nb, int nbp, int n_tok, float* y,
                     size_t y_stride, hipStream_t st);

// int8 path (kernels_i8.hip).
void launch_quantize_act(const float* x, size_t x_stride, int cols, int n_tok, int8_t* q, uint16_t* s, double* sx,
                         hipStream_t st);
void launch_gemv_i8(int dtype, const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const int8_t* aq,
                    const double* asx, int rows, int nb, int n_tok, float* y, size_t y_stride, hipStream_t st);
void launch_block_dots(int dtype, const uint8_t* qs, const int8_t* aq, int rows, int nb, int n_tok, int32_t* P,
                       hipStream_t st);

// argmax over n logits (kernels_misc.hip); partial holds 2*ceil(n/2048) words.
void launch_argmax(const float* v, size_t n, uint64_t* partial, uint64_t* out, hipStream_t st);
size_t argmax_partial_words(size_t n);

}  // namespace nnh
