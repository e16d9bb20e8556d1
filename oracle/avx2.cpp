// The timed CPU baseline: nncpu's AVX2 + FMA gemv kernels restated with the
// same intrinsics, accumulators, reduction trees and 4 KB-ahead prefetch
// (crates/nncpu/src/kernels/avx2.rs:33-108,592-642,1256-1521), run over the
// reference pool's even row split (pool.rs:318-324,413-453) with its
// threading thresholds (kernels/mod.rs:418,442,512,545).
//
// TEST INFRASTRUCTURE ONLY: used by tests/ (bit equality with the scalar
// restatement, oracle.cpp) and by bench.py's cpu_baseline leg.

#include <immintrin.h>

#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

#include "oracle.h"

namespace {

inline float bf16f(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// avx2.rs:33-40: high half onto low, then two hadds.
__attribute__((target("avx2,fma"))) inline float hsum(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(_mm_hadd_ps(s, s));
}

// avx2.rs:51-56
__attribute__((target("avx2,fma"))) inline float reduce4(__m256 a0, __m256 a1, __m256 a2, __m256 a3) {
    return hsum(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
}

// avx2.rs:65-81
__attribute__((target("avx2,fma"))) inline __m256 load_bf16(const uint16_t* p) {
    __m128i h = _mm_loadu_si128((const __m128i*)p);
    return _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
}
__attribute__((target("avx2,fma"))) inline __m256 bf16_splat(const uint16_t* p) { return _mm256_set1_ps(bf16f(*p)); }

// avx2.rs:83-108: 4 KB ahead, T1.
constexpr size_t PREFETCH_AHEAD = 4096;
__attribute__((target("avx2,fma"))) inline void prefetch(const void* p) {
    _mm_prefetch((const char*)p + PREFETCH_AHEAD, _MM_HINT_T1);
}

// avx2.rs:592-610
__attribute__((target("avx2,fma"))) float dot_bf16_raw(const uint16_t* a, const float* b, size_t n) {
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(load_bf16(a + i), _mm256_loadu_ps(b + i), acc);
    float s = hsum(acc);
    for (; i < n; ++i) {
        float p = bf16f(a[i]) * b[i];
        s = s + p;
    }
    return s;
}

// avx2.rs:628-642
__attribute__((target("avx2,fma"))) void block_sums_raw(const float* x, float* out, size_t nb) {
    for (size_t b = 0; b < nb; ++b) {
        const float* xb = x + 32 * b;
        __m256 acc = _mm256_loadu_ps(xb);
        acc = _mm256_add_ps(acc, _mm256_loadu_ps(xb + 8));
        acc = _mm256_add_ps(acc, _mm256_loadu_ps(xb + 16));
        acc = _mm256_add_ps(acc, _mm256_loadu_ps(xb + 24));
        out[b] = hsum(acc);
    }
}

// avx2.rs:1256-1263
__attribute__((target("avx2,fma"))) inline __m256 q8_widen(const int8_t* q, __m256 sc) {
    __m128i v = _mm_loadl_epi64((const __m128i*)q);
    return _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(v)), sc);
}

// avx2.rs:1265-1292
__attribute__((target("avx2,fma"))) float q8_row1(const int8_t* q, const uint16_t* s, const float* x, size_t nb) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (size_t b = 0; b < nb; ++b) {
        __m256 sc = bf16_splat(s + b);
        const int8_t* qb = q + 32 * b;
        const float* xb = x + 32 * b;
        if (b % 2 == 0) prefetch(qb);
        a0 = _mm256_fmadd_ps(q8_widen(qb, sc), _mm256_loadu_ps(xb), a0);
        a1 = _mm256_fmadd_ps(q8_widen(qb + 8, sc), _mm256_loadu_ps(xb + 8), a1);
        a2 = _mm256_fmadd_ps(q8_widen(qb + 16, sc), _mm256_loadu_ps(xb + 16), a2);
        a3 = _mm256_fmadd_ps(q8_widen(qb + 24, sc), _mm256_loadu_ps(xb + 24), a3);
    }
    return reduce4(a0, a1, a2, a3);
}

// avx2.rs:1294-1336
__attribute__((target("avx2,fma"))) void q8_row3(const int8_t* q, const uint16_t* s, const float* const* x,
                                                 size_t nb, float* out) {
    __m256 z = _mm256_setzero_ps();
    __m256 a00 = z, a01 = z, a02 = z, a03 = z, a10 = z, a11 = z, a12 = z, a13 = z, a20 = z, a21 = z, a22 = z,
           a23 = z;
    const float *x0 = x[0], *x1 = x[1], *x2 = x[2];
    for (size_t b = 0; b < nb; ++b) {
        __m256 sc = bf16_splat(s + b);
        const int8_t* qb = q + 32 * b;
        size_t o = 32 * b;
        if (b % 2 == 0) prefetch(qb);
        __m256 w = q8_widen(qb, sc);
        a00 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o), a00);
        a10 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o), a10);
        a20 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o), a20);
        w = q8_widen(qb + 8, sc);
        a01 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o + 8), a01);
        a11 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o + 8), a11);
        a21 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o + 8), a21);
        w = q8_widen(qb + 16, sc);
        a02 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o + 16), a02);
        a12 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o + 16), a12);
        a22 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o + 16), a22);
        w = q8_widen(qb + 24, sc);
        a03 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o + 24), a03);
        a13 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o + 24), a13);
        a23 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o + 24), a23);
    }
    out[0] = reduce4(a00, a01, a02, a03);
    out[1] = reduce4(a10, a11, a12, a13);
    out[2] = reduce4(a20, a21, a22, a23);
}

// avx2.rs:1377-1387
__attribute__((target("avx2,fma"))) inline void q4_bytes(const uint8_t* q, __m256i* lo, __m256i* hi) {
    *lo = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)q));
    *hi = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(q + 8)));
}
__attribute__((target("avx2,fma"))) inline __m256 q4_scale(__m256i v, __m256 sc) {
    return _mm256_mul_ps(_mm256_cvtepi32_ps(v), sc);
}

// avx2.rs:1395-1436
__attribute__((target("avx2,fma"))) float q4_row1(const uint8_t* q, const uint16_t* s, const float* x, size_t nb) {
    __m256i mask = _mm256_set1_epi32(0x0f);
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (size_t b = 0; b < nb; ++b) {
        __m256 sc = bf16_splat(s + b);
        __m256i lo, hi;
        q4_bytes(q + 16 * b, &lo, &hi);
        const float* xb = x + 32 * b;
        if (b % 4 == 0) prefetch(q + 16 * b);
        a0 = _mm256_fmadd_ps(q4_scale(_mm256_and_si256(lo, mask), sc), _mm256_loadu_ps(xb), a0);
        a1 = _mm256_fmadd_ps(q4_scale(_mm256_and_si256(hi, mask), sc), _mm256_loadu_ps(xb + 8), a1);
        a2 = _mm256_fmadd_ps(q4_scale(_mm256_srli_epi32(lo, 4), sc), _mm256_loadu_ps(xb + 16), a2);
        a3 = _mm256_fmadd_ps(q4_scale(_mm256_srli_epi32(hi, 4), sc), _mm256_loadu_ps(xb + 24), a3);
    }
    return reduce4(a0, a1, a2, a3);
}

// avx2.rs:1438-1478
__attribute__((target("avx2,fma"))) void q4_row3(const uint8_t* q, const uint16_t* s, const float* const* x,
                                                 size_t nb, float* out) {
    __m256 z = _mm256_setzero_ps();
    __m256 a00 = z, a01 = z, a02 = z, a03 = z, a10 = z, a11 = z, a12 = z, a13 = z, a20 = z, a21 = z, a22 = z,
           a23 = z;
    const float *x0 = x[0], *x1 = x[1], *x2 = x[2];
    for (size_t b = 0; b < nb; ++b) {
        __m256 sc = bf16_splat(s + b);
        __m256i lo, hi;
        q4_bytes(q + 16 * b, &lo, &hi);
        size_t o = 32 * b;
        if (b % 4 == 0) prefetch(q + 16 * b);
        __m256 w = q4_scale(_mm256_srli_epi32(_mm256_slli_epi32(lo, 28), 28), sc);
        a00 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o), a00);
        a10 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o), a10);
        a20 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o), a20);
        w = q4_scale(_mm256_srli_epi32(_mm256_slli_epi32(hi, 28), 28), sc);
        a01 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o + 8), a01);
        a11 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o + 8), a11);
        a21 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o + 8), a21);
        w = q4_scale(_mm256_srli_epi32(lo, 4), sc);
        a02 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o + 16), a02);
        a12 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o + 16), a12);
        a22 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o + 16), a22);
        w = q4_scale(_mm256_srli_epi32(hi, 4), sc);
        a03 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x0 + o + 24), a03);
        a13 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x1 + o + 24), a13);
        a23 = _mm256_fmadd_ps(w, _mm256_loadu_ps(x2 + o + 24), a23);
    }
    out[0] = reduce4(a00, a01, a02, a03);
    out[1] = reduce4(a10, a11, a12, a13);
    out[2] = reduce4(a20, a21, a22, a23);
}

// avx2.rs:1338-1375 for rows [r0, r1).
void q8_rows_raw(const int8_t* qs, const uint16_t* sc, const float* x, size_t x_stride, size_t cols, float* y,
                 size_t y_stride, size_t n_vec, size_t r0, size_t r1) {
    size_t nb = cols / 32;
    if (n_vec == 1) {
        for (size_t r = r0; r < r1; ++r) y[r] = q8_row1(qs + r * cols, sc + r * nb, x, nb);
        return;
    }
    for (size_t r = r0; r < r1; ++r) {
        const int8_t* q = qs + r * cols;
        const uint16_t* s = sc + r * nb;
        size_t n = 0;
        for (; n + 3 <= n_vec; n += 3) {
            const float* xv[3] = {x + n * x_stride, x + (n + 1) * x_stride, x + (n + 2) * x_stride};
            float o[3];
            q8_row3(q, s, xv, nb, o);
            for (int t = 0; t < 3; ++t) y[(n + t) * y_stride + r] = o[t];
        }
        for (; n < n_vec; ++n) y[n * y_stride + r] = q8_row1(q, s, x + n * x_stride, nb);
    }
}

// avx2.rs:1480-1521 for rows [r0, r1).
void q4_rows_raw(const uint8_t* qs, const uint16_t* sc, const uint16_t* bi, const float* x, size_t x_stride,
                 const float* xsum, size_t xsum_stride, size_t cols, float* y, size_t y_stride, size_t n_vec,
                 size_t r0, size_t r1) {
    size_t nb = cols / 32;
    if (n_vec == 1) {
        for (size_t r = r0; r < r1; ++r)
            y[r] = q4_row1(qs + r * cols / 2, sc + r * nb, x, nb) + dot_bf16_raw(bi + r * nb, xsum, nb);
        return;
    }
    for (size_t r = r0; r < r1; ++r) {
        const uint8_t* q = qs + r * cols / 2;
        const uint16_t* s = sc + r * nb;
        const uint16_t* b = bi + r * nb;
        size_t n = 0;
        for (; n + 3 <= n_vec; n += 3) {
            const float* xv[3] = {x + n * x_stride, x + (n + 1) * x_stride, x + (n + 2) * x_stride};
            float o[3];
            q4_row3(q, s, xv, nb, o);
            for (int t = 0; t < 3; ++t)
                y[(n + t) * y_stride + r] = o[t] + dot_bf16_raw(b, xsum + (n + t) * xsum_stride, nb);
        }
        for (; n < n_vec; ++n)
            y[n * y_stride + r] =
                q4_row1(q, s, x + n * x_stride, nb) + dot_bf16_raw(b, xsum + n * xsum_stride, nb);
    }
}

// A persistent spin pool, as pool.rs:1-10,248-295: the caller runs tid 0,
// workers spin on a generation counter, then yield.
class Pool {
public:
    void resize(int n) {
        stop_all();
        n_ = n < 1 ? 1 : n;
        quit_.store(false);
        // Each worker starts from the generation current now: a worker that
        // read it only once running could miss a dispatch issued meanwhile.
        const uint64_t g0 = gen_.load();
        for (int t = 1; t < n_; ++t) workers_.emplace_back([this, t, g0] { loop(t, g0); });
    }
    int size() const { return n_; }
    void dispatch(const std::function<void(int, int)>& f) {
        if (n_ == 1) {
            f(0, 1);
            return;
        }
        job_ = &f;
        done_.store(0, std::memory_order_relaxed);
        gen_.fetch_add(1, std::memory_order_release);
        f(0, n_);
        while (done_.load(std::memory_order_acquire) != n_ - 1) _mm_pause();
        job_ = nullptr;
    }
    ~Pool() { stop_all(); }

private:
    void loop(int tid, uint64_t seen) {
        for (;;) {
            int spins = 0;
            uint64_t g;
            while ((g = gen_.load(std::memory_order_acquire)) == seen) {
                if (quit_.load(std::memory_order_relaxed)) return;
                if (++spins < 20000)
                    _mm_pause();
                else
                    std::this_thread::yield();
            }
            seen = g;
            (*job_)(tid, n_);
            done_.fetch_add(1, std::memory_order_acq_rel);
        }
    }
    void stop_all() {
        quit_.store(true);
        for (auto& w : workers_) w.join();
        workers_.clear();
    }
    int n_ = 1;
    std::vector<std::thread> workers_;
    std::atomic<uint64_t> gen_{0};
    std::atomic<int> done_{0};
    std::atomic<bool> quit_{false};
    const std::function<void(int, int)>* volatile job_ = nullptr;
};

Pool& pool() {
    static Pool p;
    static bool init = [] {
        unsigned hw = std::thread::hardware_concurrency();
        p.resize((int)std::min(8u, hw ? hw : 1u));  // pool.rs:85-95 default
        return true;
    }();
    (void)init;
    return p;
}

// pool.rs:318-324
inline void split_range(size_t total, int tid, int n, size_t* first, size_t* last) {
    size_t per = total / n, rem = total % n;
    size_t t = (size_t)tid;
    *first = t * per + std::min(t, rem);
    *last = *first + per + (t < rem ? 1 : 0);
}

// pool.rs:413-453 with unit = 1.
void for_rows(bool threaded, size_t rows, const std::function<void(size_t, size_t)>& f) {
    if (rows == 0) return;
    if (!threaded || pool().size() == 1) {
        f(0, rows);
        return;
    }
    pool().dispatch([&](int tid, int nth) {
        size_t a, b;
        split_range(rows, tid, nth, &a, &b);
        if (a < b) f(a, b);
    });
}

}  // namespace

extern "C" {

int avx_available(void) { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }
void avx_set_threads(int n) { pool().resize(n); }
int avx_threads(void) { return pool().size(); }

// model/forward.rs:15-58 -> kernels/mod.rs:408-552 on the AVX2 backend.
int avx_gemv_batch(int dtype, const void* w, size_t rows, size_t cols, const float* x, size_t x_stride, float* y,
                   size_t y_stride, size_t n_tok) {
    if (n_tok == 0 || rows == 0 || cols == 0) return 0;
    if (cols % 32 != 0) return -1;
    size_t n = rows * cols, nb = cols / 32;
    const uint8_t* base = (const uint8_t*)w;
    bool multi = pool().size() > 1;
    bool threaded = n_tok == 1 ? (multi && rows >= 256 && cols >= 256) : (multi && rows >= 64 && cols >= 256);
    if (dtype == 1) {
        const int8_t* qs = (const int8_t*)base;
        const uint16_t* sc = (const uint16_t*)(base + n);
        for_rows(threaded, rows, [&](size_t a, size_t b) { q8_rows_raw(qs, sc, x, x_stride, cols, y, y_stride, n_tok, a, b); });
        return 0;
    }
    if (dtype == 2) {
        const uint8_t* qs = base;
        const uint16_t* sc = (const uint16_t*)(base + n / 2);
        const uint16_t* bi = sc + n / 32;
        std::vector<float> xsum(n_tok * nb);
        for (size_t t = 0; t < n_tok; ++t) block_sums_raw(x + t * x_stride, xsum.data() + t * nb, nb);
        for_rows(threaded, rows, [&](size_t a, size_t b) {
            q4_rows_raw(qs, sc, bi, x, x_stride, xsum.data(), nb, cols, y, y_stride, n_tok, a, b);
        });
        return 0;
    }
    return -1;
}

// A gemv callback for the Gemma-3 harness (nncpu_amd/host/gemma3.cpp):
// matrix `id` of a table of split-layout buffers, on the AVX2 restatement.
struct or_model_table {
    int n, dtype;
    const void* const* bufs;
    const size_t* rows;
    const size_t* cols;
};

int or_model_gemv_cb(void* ctx, int id, const float* x, size_t x_stride, float* y, size_t y_stride, size_t n_tok) {
    const or_model_table* t = (const or_model_table*)ctx;
    if (id < 0 || id >= t->n) return 1;
    return avx_gemv_batch(t->dtype, t->bufs[id], t->rows[id], t->cols[id], x, x_stride, y,
                          n_tok > 1 ? y_stride : t->rows[id], n_tok) != 0;
}

// The reference's "load-only roofline" calibration (kernels/tests.rs:1306-1321):
// one thread streams a buffer with almost no work per byte; best of reps.
__attribute__((target("avx2,fma"))) double avx_stream_gbs(size_t bytes, int reps) {
    size_t n = bytes / 4 / 32 * 32;
    std::vector<float> big(n);
    for (size_t i = 0; i < n; ++i) big[i] = (float)(i & 255);
    double best = 1e30;
    volatile float sink = 0;
    for (int r = 0; r <= reps; ++r) {
        auto t0 = std::chrono::steady_clock::now();
        __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
        for (size_t i = 0; i < n; i += 32) {
            a0 = _mm256_fmadd_ps(_mm256_loadu_ps(&big[i]), _mm256_loadu_ps(&big[i]), a0);
            a1 = _mm256_fmadd_ps(_mm256_loadu_ps(&big[i + 8]), _mm256_loadu_ps(&big[i + 8]), a1);
            a2 = _mm256_fmadd_ps(_mm256_loadu_ps(&big[i + 16]), _mm256_loadu_ps(&big[i + 16]), a2);
            a3 = _mm256_fmadd_ps(_mm256_loadu_ps(&big[i + 24]), _mm256_loadu_ps(&big[i + 24]), a3);
        }
        sink = sink + reduce4(a0, a1, a2, a3);
        double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        if (r > 0 && dt < best) best = dt;  // r == 0 is the warm-up
    }
    return (double)(n * 4) / best / 1e9;
}

}  // extern "C"
