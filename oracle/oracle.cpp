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

// ---- GGUF block decoding (kernels/quant.rs:97-291), the load-time step ----

namespace {

// runtime.rs:25-48: IEEE half -> f32 by bits (subnormals renormalised, NaN
// payloads kept).
float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int e = 127 - 15 + 1;
            uint32_t m = mant;
            while (!(m & 0x400)) {
                m <<= 1;
                e -= 1;
            }
            bits = sign | ((uint32_t)e << 23) | ((m & 0x3ff) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float f16_at(const uint8_t* b, size_t i) { return f16_to_f32((uint16_t)(b[i] | (b[i + 1] << 8))); }

// quant.rs:163-195: Q4_0 / Q4_1 / Q5_0 / Q5_1 (optional fp16 min, optional
// fifth bit per value; centred on 8, or 16 with the fifth bit, when no min).
void dequant_legacy(const uint8_t* src, size_t nblocks, bool has_min, bool has_high, float* dst) {
    const size_t bytes = 2 + (has_min ? 2 : 0) + (has_high ? 4 : 0) + 16;
    const int centre = has_min ? 0 : has_high ? 16 : 8;
    for (size_t bi = 0; bi < nblocks; ++bi) {
        const uint8_t* p = src + bi * bytes;
        float* y = dst + 32 * bi;
        const float d = f16_at(p, 0), m = has_min ? f16_at(p, 2) : 0.0f;
        const size_t o = has_min ? 4 : 2;
        const uint32_t qh = has_high ? (uint32_t)p[o] | (uint32_t)p[o + 1] << 8 | (uint32_t)p[o + 2] << 16 |
                                           (uint32_t)p[o + 3] << 24
                                     : 0u;
        const uint8_t* qs = p + bytes - 16;
        for (int j = 0; j < 16; ++j) {
            const int hi0 = (int)(((qh >> j) << 4) & 0x10), hi1 = (int)((qh >> (j + 12)) & 0x10);
            y[j] = (float)(((int)(qs[j] & 0x0f) | hi0) - centre) * d + m;
            y[j + 16] = (float)(((int)(qs[j] >> 4) | hi1) - centre) * d + m;
        }
    }
}

// quant.rs:197-211 (ggml's packing of 6-bit scales and mins).
void scale_min_k4(int j, const uint8_t* q, float* d, float* m) {
    uint8_t dd, mm;
    if (j < 4) {
        dd = q[j] & 63;
        mm = q[j + 4] & 63;
    } else {
        dd = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        mm = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
    *d = (float)dd;
    *m = (float)mm;
}

// quant.rs:213-236 (Q4_K) and :238-266 (Q5_K, qh with each value's fifth bit).
void dequant_qk(const uint8_t* src, size_t nblocks, bool q5, float* dst) {
    const size_t bytes = q5 ? 176 : 144;
    for (size_t bi = 0; bi < nblocks; ++bi) {
        const uint8_t* b = src + bi * bytes;
        float* y = dst + 256 * bi;
        const float d = f16_at(b, 0), dmin = f16_at(b, 2);
        const uint8_t* scales = b + 4;
        const uint8_t* qh = b + 16;
        const uint8_t* qs = b + (q5 ? 48 : 16);
        uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < 4; ++j) {
            float sc, mn;
            scale_min_k4(2 * j, scales, &sc, &mn);
            const float d1 = d * sc, m1 = dmin * mn;
            scale_min_k4(2 * j + 1, scales, &sc, &mn);
            const float d2 = d * sc, m2 = dmin * mn;
            const uint8_t* q = qs + 32 * j;
            for (int l = 0; l < 32; ++l) {
                const int h1 = q5 && (qh[l] & u1) ? 16 : 0, h2 = q5 && (qh[l] & u2) ? 16 : 0;
                y[64 * j + l] = d1 * (float)((q[l] & 0x0f) + h1) - m1;
                y[64 * j + l + 32] = d2 * (float)((q[l] >> 4) + h2) - m2;
            }
            u1 = (uint8_t)(u1 << 2);
            u2 = (uint8_t)(u2 << 2);
        }
    }
}

// quant.rs:268-291 (Q6_K: 4 low bits in ql, 2 high bits in qh, an int8
// scale per 16 values).
void dequant_q6k(const uint8_t* src, size_t nblocks, float* dst) {
    for (size_t bi = 0; bi < nblocks; ++bi) {
        const uint8_t* b = src + bi * 210;
        const float d = f16_at(b, 208);
        for (int h = 0; h < 2; ++h) {
            const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
            const int8_t* sc = (const int8_t*)(b + 192 + 8 * h);
            float* y = dst + 256 * bi + 128 * h;
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0x0f) | ((qh[l] & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l] = d * (float)sc[is] * (float)q1;
                y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                y[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

}  // namespace

// gguf.rs:335-355 for the decodable types: bytes and elements per block.
int or_ggml_block(uint32_t t, size_t* bytes, size_t* per) {
    switch (t) {
        case 0: *bytes = 4, *per = 1; return 1;
        case 1: *bytes = 2, *per = 1; return 1;
        case 30: *bytes = 2, *per = 1; return 1;
        case 2: *bytes = 18, *per = 32; return 1;
        case 3: *bytes = 20, *per = 32; return 1;
        case 6: *bytes = 22, *per = 32; return 1;
        case 7: *bytes = 24, *per = 32; return 1;
        case 8: *bytes = 34, *per = 32; return 1;
        case 12: *bytes = 144, *per = 256; return 1;
        case 13: *bytes = 176, *per = 256; return 1;
        case 14: *bytes = 210, *per = 256; return 1;
        default: return 0;
    }
}

// quant.rs:107-156 (dequantize_to_f32): 0 (dst untouched) for other types,
// when n is not a whole number of blocks or blocks holds fewer than needed.
int or_dequantize_to_f32(uint32_t t, const uint8_t* blocks, size_t nbytes, float* dst, size_t n) {
    size_t bytes, per;
    if (!or_ggml_block(t, &bytes, &per)) return 0;
    if (n % per != 0 || nbytes / bytes < n / per) return 0;
    const size_t nb = n / per;
    switch (t) {
        case 0:
            std::memcpy(dst, blocks, 4 * n);
            break;
        case 1:
            for (size_t i = 0; i < n; ++i) dst[i] = f16_at(blocks, 2 * i);
            break;
        case 30:
            for (size_t i = 0; i < n; ++i) dst[i] = bf16_to_f32((uint16_t)(blocks[2 * i] | (blocks[2 * i + 1] << 8)));
            break;
        case 8:
            for (size_t bi = 0; bi < nb; ++bi) {
                const uint8_t* b = blocks + 34 * bi;
                const float d = f16_at(b, 0);
                for (int k = 0; k < 32; ++k) dst[32 * bi + k] = d * (float)(int8_t)b[2 + k];
            }
            break;
        case 2: dequant_legacy(blocks, nb, false, false, dst); break;
        case 3: dequant_legacy(blocks, nb, true, false, dst); break;
        case 6: dequant_legacy(blocks, nb, false, true, dst); break;
        case 7: dequant_legacy(blocks, nb, true, true, dst); break;
        case 12: dequant_qk(blocks, nb, false, dst); break;
        case 13: dequant_qk(blocks, nb, true, dst); break;
        case 14: dequant_q6k(blocks, nb, dst); break;
    }
    return 1;
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
