// Seeded synthetic data for the config-1 model: the reference's test
// generator (crates/nncpu/src/kernels/tests.rs:9-50, xorshift64* with
// Box-Muller normals), run over fixed-size chunks of a tensor, each chunk
// from its own seed, so a large tensor is drawn on many threads and is the
// same whatever the thread count.

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

namespace {

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s((seed * 0x9e3779b97f4a7c15ull) | 1ull) {}  // tests.rs:13-15
    uint64_t next() {                                                           // tests.rs:17-22
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 0x2545f4914f6cdd1dull;
    }
    float unit() { return (float)(next() >> 40) / (float)(1ull << 24); }  // tests.rs:25-27
    float normal() {                                                      // tests.rs:33-37
        float u1 = unit();
        u1 = u1 > 1e-7f ? u1 : 1e-7f;
        const float u2 = unit();
        return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
    }
};

}  // namespace

extern "C" {

// out[i] = mean + sd * normal, element i drawn as element i % chunk of the
// generator seeded with seed + i / chunk (tests.rs:44-46 per chunk).
void nng_rng_normals(uint64_t seed, size_t n, float mean, float sd, size_t chunk, int threads, float* out) {
    if (chunk == 0) chunk = n ? n : 1;
    const size_t nchunks = (n + chunk - 1) / chunk;
    if (threads < 1) threads = 1;
    auto work = [&](int tid) {
        for (size_t c = (size_t)tid; c < nchunks; c += (size_t)threads) {
            Rng r(seed + c);
            const size_t end = (c + 1) * chunk < n ? (c + 1) * chunk : n;
            for (size_t i = c * chunk; i < end; ++i) {
                const float z = sd * r.normal();
                out[i] = mean == 0.0f ? z : mean + z;
            }
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; ++t) pool.emplace_back(work, t);
    work(0);
    for (auto& t : pool) t.join();
}

}  // extern "C"
