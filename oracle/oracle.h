// CPU oracle for nncpu's quantized matmul: TEST INFRASTRUCTURE ONLY (see
// oracle.cpp's header). Declarations of the scalar restatement
// (oracle.cpp) and the timed AVX2 restatement (avx2.cpp).
#pragma once
#include <cstddef>
#include <cstdint>

extern "C" {

float or_bf16_to_f32(uint16_t v);
uint16_t or_f32_to_bf16(float f);
int32_t or_rint(float v);

void or_quantize_q8_0(const float* src, size_t n, int8_t* qs, uint16_t* scales);
void or_quantize_q4(const float* src, size_t n, uint8_t* qs, uint16_t* scales, uint16_t* biases);
void or_block_sums(const float* x, size_t n, float* out);
float or_dot_bf16_f32(const uint16_t* a, const float* b, size_t n);

void or_gemv_q8_0_rows(const int8_t* qs, const uint16_t* scales, const float* x, size_t x_stride, size_t cols,
                       float* y, size_t y_stride, size_t n_vec, size_t r0, size_t r1);
void or_gemv_q4_rows(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const float* x,
                     size_t x_stride, const float* xsum, size_t xsum_stride, size_t cols, float* y,
                     size_t y_stride, size_t n_vec, size_t r0, size_t r1);
int or_gemv_q8_0_batch(const int8_t* qs, const uint16_t* scales, const float* x, size_t x_stride, float* y,
                       size_t y_stride, size_t rows, size_t cols, size_t n_batch);
int or_gemv_q4_batch(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const float* x,
                     size_t x_stride, const float* xsum, size_t xsum_stride, float* y, size_t y_stride,
                     size_t rows, size_t cols, size_t n_batch);
int or_gemv_batch(int dtype, const void* w, size_t rows, size_t cols, const float* x, size_t x_stride, float* y,
                  size_t y_stride, size_t n_tok);
size_t or_argmax(const float* v, size_t n);

void or_gemv_bf16(const uint16_t* w, const float* x, float* y, size_t rows, size_t cols);
void or_gemv_bf16_batch(const uint16_t* w, const float* x, size_t x_stride, float* y, size_t y_stride, size_t rows,
                        size_t cols, size_t n_batch);
size_t or_gemv_bf16_argmax(const uint16_t* w, const float* x, size_t rows, size_t cols);

int or_ggml_block(uint32_t t, size_t* bytes, size_t* per);
int or_dequantize_to_f32(uint32_t t, const uint8_t* blocks, size_t nbytes, float* dst, size_t n);

void or_block_dots(int dtype, const void* qs, size_t rows, size_t cols, const int8_t* qx, int32_t* P);
void or_dequant_act(const int8_t* qx, const uint16_t* sx, size_t n, float* out);
void or_gemv_i8_exact(int dtype, const void* w, size_t rows, size_t cols, const int8_t* qx, const uint16_t* sx,
                      float* y);

void or_rng_init(uint64_t* state, uint64_t seed);
uint64_t or_rng_next(uint64_t* state);
void or_rng_uniform(uint64_t* st, size_t n, float lo, float hi, float* out);
void or_rng_normals(uint64_t* st, size_t n, float sd, float* out);

// avx2.cpp: the AVX2 kernels with the reference's row split over a pool.
int avx_available(void);
void avx_set_threads(int n);
int avx_threads(void);
int avx_gemv_batch(int dtype, const void* w, size_t rows, size_t cols, const float* x, size_t x_stride, float* y,
                   size_t y_stride, size_t n_tok);
double avx_stream_gbs(size_t bytes, int reps);
int or_model_gemv_cb(void* ctx, int id, const float* x, size_t x_stride, float* y, size_t y_stride, size_t n_tok);
}
