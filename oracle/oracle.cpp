// CPU oracle for the nncpu quantized-matmul path.
//
// TEST INFRASTRUCTURE ONLY. Nothing in the product (nncpu_amd/, include/)
// links, loads or calls this file. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg use it, and only as the checker or the timed
// CPU baseline, never as the thing measured on the GPU.
//
// A scalar C++ restatement of nncpu's portable kernels, lane by lane, in the
// reference's exact operation order. Build flags: -O2 -ffp-contract=off
// -mfma, so that a*b+c is never fused by the compiler and std::fma is the
// one fused multiply-add, used exactly where the reference's `fmadd`
// (crates/nncpu/src/kernels/scalar.rs:46-54) and `_mm256_fmadd_ps`
// (kernels/avx2.rs) fuse.
//
// Parity pins (tests/test_oracle.py): the reference's own known-answer tests
// (kernels/tests.rs:502-553,578-614; runtime.rs:225-241;
// model/tests.rs:404-423), f64 brute force, closed forms, the batch == single
// and thread-count invariances, and scalar == AVX2 bit equality (oracle/avx2.cpp).

#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstddef>
#include <algorithm>
#include <vector>

#include "oracle.h"

namespace {

// runtime.rs:10-13
inline float bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// runtime.rs:15-21, round to nearest even via the 0x7fff bias.
inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    uint32_t rounding_bias = 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)((u + rounding_bias) >> 16);
}

// quant.rs:13-16
inline float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// Rust's saturating `f32 as i32`: NaN -> 0, out of range -> the bound.
inline int32_t sat_i32(float v) {
    if (std::isnan(v)) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

// quant.rs:18-29 (`lrintf`, ties to even).
inline int32_t rint_i32(float v) {
    const float MAGIC = 12582912.0f;  // 1.5 * 2^23
    if (std::fabs(v) < 4194304.0f) {
        volatile float t = v + MAGIC;  // volatile: keep the two roundings
        return (int32_t)(t - MAGIC);
    }
    return sat_i32(std::nearbyint(v));
}

typedef float V8[8];

// scalar.rs:108-117
inline float hsum8(const float* v) {
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// scalar.rs:626-649: the Q8_0 row kernel for N tokens.
template <int N>
void q8_row(const int8_t* q, const uint16_t* s, size_t nb, const float* const* xs, float* out) {
    float acc[N][4][8] = {};
    for (size_t b = 0; b < nb; ++b) {
        const int8_t* qb = q + 32 * b;
        float sc = bf16_to_f32(s[b]);
        for (int k = 0; k < 4; ++k) {
            float w[8];
            for (int l = 0; l < 8; ++l) w[l] = (float)qb[8 * k + l] * sc;
            for (int t = 0; t < N; ++t) {
                const float* xt = xs[t] + 32 * b + 8 * k;
                for (int l = 0; l < 8; ++l) acc[t][k][l] = std::fma(w[l], xt[l], acc[t][k][l]);
            }
        }
    }
    for (int t = 0; t < N; ++t) {
        float v[8];
        for (int l = 0; l < 8; ++l) v[l] = (acc[t][0][l] + acc[t][1][l]) + (acc[t][2][l] + acc[t][3][l]);
        out[t] = hsum8(v);
    }
}

// scalar.rs:651-674: the Q4 row kernel for N tokens (bias term excluded).
template <int N>
void q4_row(const uint8_t* q, const uint16_t* s, size_t nb, const float* const* xs, float* out) {
    float acc[N][4][8] = {};
    for (size_t b = 0; b < nb; ++b) {
        const uint8_t* qb = q + 16 * b;
        float sc = bf16_to_f32(s[b]);
        float w[4][8];
        for (int l = 0; l < 8; ++l) {
            w[0][l] = (float)(qb[l] & 15) * sc;
            w[1][l] = (float)(qb[8 + l] & 15) * sc;
            w[2][l] = (float)(qb[l] >> 4) * sc;
            w[3][l] = (float)(qb[8 + l] >> 4) * sc;
        }
        for (int t = 0; t < N; ++t) {
            for (int k = 0; k < 4; ++k) {
                const float* xt = xs[t] + 32 * b + 8 * k;
                for (int l = 0; l < 8; ++l) acc[t][k][l] = std::fma(w[k][l], xt[l], acc[t][k][l]);
            }
        }
    }
    for (int t = 0; t < N; ++t) {
        float v[8];
        for (int l = 0; l < 8; ++l) v[l] = (acc[t][0][l] + acc[t][1][l]) + (acc[t][2][l] + acc[t][3][l]);
        out[t] = hsum8(v);
    }
}

// scalar.rs:334-347: one 8-lane accumulator, hsum8, then an unfused tail.
float dot_bf16_f32_impl(const uint16_t* a, const float* b, size_t n) {
    size_t body = n & ~(size_t)7;
    float acc[8] = {};
    for (size_t i = 0; i < body; i += 8)
        for (int l = 0; l < 8; ++l) acc[l] = std::fma(bf16_to_f32(a[i + l]), b[i + l], acc[l]);
    float s = hsum8(acc);
    for (size_t i = body; i < n; ++i) {
        float p = bf16_to_f32(a[i]) * b[i];
        s = s + p;
    }
    return s;
}

}  // namespace

extern "C" {

float or_bf16_to_f32(uint16_t v) { return bf16_to_f32(v); }
uint16_t or_f32_to_bf16(float f) { return f32_to_bf16(f); }
int32_t or_rint(float v) { return rint_i32(v); }

// quant.rs:31-60
void or_quantize_q8_0(const float* src, size_t n, int8_t* qs, uint16_t* scales) {
    for (size_t blk = 0; blk < n / 32; ++blk) {
        const float* b = src + 32 * blk;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i)
            if (std::fabs(b[i]) > amax) amax = std::fabs(b[i]);
        // Times the reciprocal of 127, as the reference does.
        float scale = bf16_round(amax * (1.0f / 127.0f));
        scales[blk] = f32_to_bf16(scale);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int i = 0; i < 32; ++i) qs[32 * blk + i] = (int8_t)clampi(rint_i32(b[i] * inv), -127, 127);
    }
}

// quant.rs:62-95
void or_quantize_q4(const float* src, size_t n, uint8_t* qs, uint16_t* scales, uint16_t* biases) {
    for (size_t blk = 0; blk < n / 32; ++blk) {
        const float* b = src + 32 * blk;
        float lo = b[0], hi = b[0];
        for (int i = 1; i < 32; ++i) {
            if (b[i] < lo) lo = b[i];
            if (b[i] > hi) hi = b[i];
        }
        float scale = bf16_round((hi - lo) * (1.0f / 15.0f));
        float bias = bf16_round(lo);
        scales[blk] = f32_to_bf16(scale);
        biases[blk] = f32_to_bf16(bias);
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int k = 0; k < 16; ++k) {
            int32_t q0 = clampi(rint_i32((b[k] - bias) * inv), 0, 15);
            int32_t q1 = clampi(rint_i32((b[k + 16] - bias) * inv), 0, 15);
            qs[16 * blk + k] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// scalar.rs:355-359
void or_block_sums(const float* x, size_t n, float* out) {
    for (size_t b = 0; b < n / 32; ++b) {
        const float* c = x + 32 * b;
        float v[8];
        for (int l = 0; l < 8; ++l) v[l] = ((c[l] + c[8 + l]) + c[16 + l]) + c[24 + l];
        out[b] = hsum8(v);
    }
}

float or_dot_bf16_f32(const uint16_t* a, const float* b, size_t n) { return dot_bf16_f32_impl(a, b, n); }

// scalar.rs:676-704 for rows [r0, r1) (`gemv_q8_0_rows`): tokens three at a
// time, then one by one.
void or_gemv_q8_0_rows(const int8_t* qs, const uint16_t* scales, const float* x, size_t x_stride,
                       size_t cols, float* y, size_t y_stride, size_t n_vec, size_t r0, size_t r1) {
    size_t nb = cols / 32;
    for (size_t r = r0; r < r1; ++r) {
        const int8_t* q = qs + r * cols;
        const uint16_t* s = scales + r * nb;
        size_t n = 0;
        while (n + 3 <= n_vec) {
            const float* xv[3] = {x + n * x_stride, x + (n + 1) * x_stride, x + (n + 2) * x_stride};
            float o[3];
            q8_row<3>(q, s, nb, xv, o);
            for (int t = 0; t < 3; ++t) y[(n + t) * y_stride + r] = o[t];
            n += 3;
        }
        for (; n < n_vec; ++n) {
            const float* xv[1] = {x + n * x_stride};
            float o[1];
            q8_row<1>(q, s, nb, xv, o);
            y[n * y_stride + r] = o[0];
        }
    }
}

// scalar.rs:706-742 (`gemv_q4_rows`): each row's sum plus dot(biases, xsum).
void or_gemv_q4_rows(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const float* x,
                     size_t x_stride, const float* xsum, size_t xsum_stride, size_t cols, float* y,
                     size_t y_stride, size_t n_vec, size_t r0, size_t r1) {
    size_t nb = cols / 32;
    for (size_t r = r0; r < r1; ++r) {
        const uint8_t* q = qs + r * cols / 2;
        const uint16_t* s = scales + r * nb;
        const uint16_t* bi = biases + r * nb;
        size_t n = 0;
        while (n + 3 <= n_vec) {
            const float* xv[3] = {x + n * x_stride, x + (n + 1) * x_stride, x + (n + 2) * x_stride};
            float o[3];
            q4_row<3>(q, s, nb, xv, o);
            for (int t = 0; t < 3; ++t)
                y[(n + t) * y_stride + r] = o[t] + dot_bf16_f32_impl(bi, xsum + (n + t) * xsum_stride, nb);
            n += 3;
        }
        for (; n < n_vec; ++n) {
            const float* xv[1] = {x + n * x_stride};
            float o[1];
            q4_row<1>(q, s, nb, xv, o);
            y[n * y_stride + r] = o[0] + dot_bf16_f32_impl(bi, xsum + n * xsum_stride, nb);
        }
    }
}

// kernels/mod.rs:408-423 + 487-516: the single and batched Q8_0 gemv. The
// single path is the batch path at n_batch == 1 (kernels/mod.rs:502-504).
// Returns 0, or -1 for a violated precondition (the reference panics).
int or_gemv_q8_0_batch(const int8_t* qs, const uint16_t* scales, const float* x, size_t x_stride, float* y,
                       size_t y_stride, size_t rows, size_t cols, size_t n_batch) {
    if (rows == 0 || cols == 0 || n_batch == 0) return 0;
    if (cols % 32 != 0) return -1;
    if (n_batch > 1 && y_stride < rows) return -1;
    or_gemv_q8_0_rows(qs, scales, x, x_stride, cols, y, y_stride, n_batch, 0, rows);
    return 0;
}

// kernels/mod.rs:425-446 + 518-552.
int or_gemv_q4_batch(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const float* x,
                     size_t x_stride, const float* xsum, size_t xsum_stride, float* y, size_t y_stride,
                     size_t rows, size_t cols, size_t n_batch) {
    if (rows == 0 || cols == 0 || n_batch == 0) return 0;
    if (cols % 32 != 0) return -1;
    if (n_batch > 1 && y_stride < rows) return -1;
    or_gemv_q4_rows(qs, scales, biases, x, x_stride, xsum, xsum_stride, cols, y, y_stride, n_batch, 0, rows);
    return 0;
}

// model/forward.rs:15-58 (`gemv_batch`) for a Q8_0 or Q4 tensor: the Q4
// branch first takes every token's block sums. dtype: 1 = Q8_0, 2 = Q4.
// `w` points at the split layout (runtime.rs:136-164).
int or_gemv_batch(int dtype, const void* w, size_t rows, size_t cols, const float* x, size_t x_stride,
                  float* y, size_t y_stride, size_t n_tok) {
    if (n_tok == 0 || rows == 0 || cols == 0) return 0;
    if (cols % 32 != 0) return -1;
    size_t n = rows * cols, nb = cols / 32;
    const uint8_t* base = (const uint8_t*)w;
    if (dtype == 1) {
        const int8_t* qs = (const int8_t*)base;
        const uint16_t* sc = (const uint16_t*)(base + n);
        return or_gemv_q8_0_batch(qs, sc, x, x_stride, y, y_stride, rows, cols, n_tok);
    }
    if (dtype == 2) {
        const uint8_t* qs = base;
        const uint16_t* sc = (const uint16_t*)(base + n / 2);
        const uint16_t* bi = sc + n / 32;
        std::vector<float> xsum(n_tok * nb);
        for (size_t t = 0; t < n_tok; ++t) or_block_sums(x + t * x_stride, cols, xsum.data() + t * nb);
        return or_gemv_q4_batch(qs, sc, bi, x, x_stride, xsum.data(), nb, y, y_stride, rows, cols, n_tok);
    }
    return -1;
}

// model/forward.rs:1003-1011: the first largest value; NaN never wins.
size_t or_argmax(const float* v, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; ++i)
        if (v[i] > v[best]) best = i;
    return best;
}

// ---- BF16 weights (DType::BF16, WeightFormat::Bf16) ----

namespace {

// scalar.rs:555-571: four rows, one 8-lane accumulator each over k += 8 (the
// x tile shared by the four rows), reduced ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7))
// (the hadd tree, avx2.rs:1146-1178).
void bf16_4rows(const uint16_t* w, size_t cols, const float* x, float* out) {
    float acc[4][8] = {};
    for (size_t k = 0; k < cols; k += 8)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 8; ++l)
                acc[j][l] = std::fma(bf16_to_f32(w[j * cols + k + l]), x[k + l], acc[j][l]);
    for (int j = 0; j < 4; ++j) {
        const float* a = acc[j];
        out[j] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    }
}

// scalar.rs:573-591: one row; four accumulators over 32-element strides
// when cols % 32 == 0 (add8(add8(a0, a1), add8(a2, a3)) then hsum8), else one
// (hsum8). Reached only with cols % 8 == 0.
float bf16_row(const uint16_t* w, const float* x, size_t cols) {
    if (cols % 32 == 0) {
        float acc[4][8] = {};
        for (size_t k = 0; k < cols; k += 32)
            for (int j = 0; j < 4; ++j)
                for (int l = 0; l < 8; ++l)
                    acc[j][l] = std::fma(bf16_to_f32(w[k + 8 * j + l]), x[k + 8 * j + l], acc[j][l]);
        float v[8];
        for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
        return hsum8(v);
    }
    float a[8] = {};
    for (size_t k = 0; k + 8 <= cols; k += 8)
        for (int l = 0; l < 8; ++l) a[l] = std::fma(bf16_to_f32(w[k + l]), x[k + l], a[l]);
    return hsum8(a);
}

}  // namespace

// kernels/mod.rs:337-360 (gemv_bf16) with gemv_bf16_f64 (mod.rs:556-564) for
// cols % 8 != 0, the 4-row kernel when rows % 4 == 0, else the 1-row kernel.
// The thread split (for_rows) never changes a row's arithmetic.
void or_gemv_bf16(const uint16_t* w, const float* x, float* y, size_t rows, size_t cols) {
    if (rows == 0 || cols == 0) return;
    if (cols % 8 != 0) {
        for (size_t r = 0; r < rows; ++r) {
            double s = 0.0;
            for (size_t k = 0; k < cols; ++k) s += (double)bf16_to_f32(w[r * cols + k]) * (double)x[k];
            y[r] = (float)s;
        }
        return;
    }
    if (rows % 4 == 0) {
        for (size_t r = 0; r < rows; r += 4) bf16_4rows(w + r * cols, cols, x, y + r);
        return;
    }
    for (size_t r = 0; r < rows; ++r) y[r] = bf16_row(w + r * cols, x, cols);
}

// kernels/mod.rs:454-485 (gemv_bf16_batch): every vector gets the bits of the
// single-vector gemv (the 4-row kernel per token when rows % 4 == 0 and
// cols % 8 == 0, else the single gemv per token).
void or_gemv_bf16_batch(const uint16_t* w, const float* x, size_t x_stride, float* y, size_t y_stride, size_t rows,
                        size_t cols, size_t n_batch) {
    for (size_t t = 0; t < n_batch; ++t) or_gemv_bf16(w, x + t * x_stride, y + t * y_stride, rows, cols);
}

// kernels/mod.rs:362-406 (gemv_bf16_argmax): with rows % 4 == 0 and
// cols % 8 == 0 a running best from -inf over the 4-row kernel's outputs
// (scalar.rs:612-628: `v > bv`, so NaN and -inf never win, ties go to the
// lower row, nothing taken gives 0); otherwise the gemv and the first-max
// argmax (forward.rs:1003-1011).
size_t or_gemv_bf16_argmax(const uint16_t* w, const float* x, size_t rows, size_t cols) {
    if (rows == 0 || cols == 0) return 0;
    std::vector<float> y(rows);
    or_gemv_bf16(w, x, y.data(), rows, cols);
    if (rows % 4 != 0 || cols % 8 != 0) return or_argmax(y.data(), rows);
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t r = 0; r < rows; ++r)
        if (y[r] > bv) {
            bv = y[r];
            best = r;
        }
    return best;
}

// ---- int8-activation path (new in this build; no reference counterpart) ----

// Exact int32 block dots P[r*nb + b] = sum_k q_w[r, 32b+k] * q_x[32b+k] for
// one activation vector, by brute force. Q8_0 weights are signed; Q4 nibbles
// are unsigned (element k of a block: low nibble of byte k for k < 16, high
// nibble of byte k-16 otherwise, runtime.rs:58-62).
void or_block_dots(int dtype, const void* qs, size_t rows, size_t cols, const int8_t* qx, int32_t* P) {
    size_t nb = cols / 32;
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < nb; ++b) {
            int32_t acc = 0;
            for (int k = 0; k < 32; ++k) {
                int32_t w;
                if (dtype == 1) {
                    w = ((const int8_t*)qs)[r * cols + 32 * b + k];
                } else {
                    uint8_t byte = ((const uint8_t*)qs)[r * cols / 2 + 16 * b + (k & 15)];
                    w = k < 16 ? (byte & 15) : (byte >> 4);
                }
                acc += w * (int32_t)qx[32 * b + k];
            }
            P[r * nb + b] = acc;
        }
}

// The dequantized activation x'[k] = q_x[k] * bf16(s_x[k/32]), exact in f32:
// what the reference CPU kernel is fed on the int8 path.
void or_dequant_act(const int8_t* qx, const uint16_t* sx, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)qx[i] * bf16_to_f32(sx[i / 32]);
}

// y = sum over blocks of the exact block terms, accumulated in long double
// and rounded once to f32: the value the int8 path approximates to well
// under an f32 ulp. Per block: s_w*s_x*P (+ bias*xsum for Q4), with
// xsum = s_x * sum(q_x) exact.
void or_gemv_i8_exact(int dtype, const void* w, size_t rows, size_t cols, const int8_t* qx,
                      const uint16_t* sx, float* y) {
    size_t n = rows * cols, nb = cols / 32;
    const uint8_t* base = (const uint8_t*)w;
    std::vector<int32_t> P(rows * nb);
    or_block_dots(dtype, base, rows, cols, qx, P.data());
    const uint16_t* sc = (const uint16_t*)(base + (dtype == 1 ? n : n / 2));
    const uint16_t* bi = sc + n / 32;
    for (size_t r = 0; r < rows; ++r) {
        long double acc = 0.0L;
        for (size_t b = 0; b < nb; ++b) {
            long double s = (long double)bf16_to_f32(sc[r * nb + b]) * (long double)bf16_to_f32(sx[b]);
            acc += s * (long double)P[r * nb + b];
            if (dtype == 2) {
                int32_t qsum = 0;
                for (int k = 0; k < 32; ++k) qsum += qx[32 * b + k];
                acc += (long double)bf16_to_f32(bi[r * nb + b]) * (long double)bf16_to_f32(sx[b]) *
                       (long double)qsum;
            }
        }
        y[r] = (float)(double)acc;
    }
}

// ---- deterministic test data: kernels/tests.rs:9-50 (xorshift64*) ----

void or_rng_init(uint64_t* state, uint64_t seed) { *state = (seed * 0x9e3779b97f4a7c15ull) | 1ull; }

uint64_t or_rng_next(uint64_t* state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545f4914f6cdd1dull;
}

static inline float rng_unit(uint64_t* st) {
    return (float)(or_rng_next(st) >> 40) / (float)(1ull << 24);
}

void or_rng_uniform(uint64_t* st, size_t n, float lo, float hi, float* out) {
    for (size_t i = 0; i < n; ++i) {
        float u = rng_unit(st);
        out[i] = lo + (hi - lo) * u;
    }
}

void or_rng_normals(uint64_t* st, size_t n, float sd, float* out) {
    const float TAU = 6.28318530717958647692f;
    for (size_t i = 0; i < n; ++i) {
        float u1 = std::max(rng_unit(st), 1e-7f);
        float u2 = rng_unit(st);
        float z = std::sqrt(-2.0f * std::log(u1)) * std::cos(TAU * u2);
        out[i] = sd * z;
    }
}

}  // extern "C"
