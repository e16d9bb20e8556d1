// The Gemma-3 decode step resident on the GPU: the forward of gemma3.cpp
// (crates/nncpu/src/model/forward.rs:197-439, 719-965 with the scalar.rs
// non-matmul kernels) for one token, every operation in the same order and
// rounding as that CPU restatement, so a decode gives the same tokens and
// the same per-layer hidden states bit for bit.
//
// One persistent kernel runs every layer of a step; the lm_head argmax (the
// library's nnh_model_argmax_dev) and a one-thread step end follow. The
// three are captured once in a HIP graph and replayed per token: no host
// round trip inside the decode loop.
//
// The step kernel: one workgroup of 1024 threads per CU, launched
// cooperatively (every workgroup resident at once). Workgroups 0 .. A-1
// run the attention, PK_S per query head (each computes all of its head's
// scores and HD / PK_S output elements); the others, the matmul workgroups,
// each run a share of the rows of every matmul. Per layer:
//   P0  the previous layer's post-FFW RMSNorm and residual add (layer 0:
//       the embedding row), the attention RMSNorm, q / k / v rows;
//   P1  (attention workgroups) q / k RMSNorm, NeoX RoPE, the K/V append,
//       the attention over the cached keys block by block;
//   P2  rows of the output projection;
//   P3  the post-attention RMSNorm and residual add, the FFN RMSNorm,
//       gate and up rows, GELU(gate) * up;
//   P4  rows of the down projection.
// Every matmul workgroup computes the norms itself (the same operations, so
// the same bits) and keeps the residual stream in registers.
//
// Hand-offs: every value a phase produces is stored as 64 bits, the float
// and a tag naming the step and the layer, by a relaxed device-scope atomic
// store; its consumers poll the tagged values until every tag is current.
// A value is visible exactly when its tag is: no barrier, no fence. Each
// buffer is written once per layer; before a phase of layer l + 1 can
// overwrite a buffer, every reader of layer l's values has produced an
// output that the writer transitively waited for (every matmul workgroup
// has rows in every phase, which nngd_create checks). Every poll is
// bounded: a wait that runs out sets the error flag, which ends every other
// wait too, so every wave exits.
//
// Weights: a matmul workgroup's rows of each matrix (the 16-lane quant
// layout of the library's Q8_0 f32 path, the BF16 scale rows and, for Q4,
// the bias rows) are copied into LDS by direct global->LDS loads one layer
// ahead: layer l + 1's q / k / v rows as soon as layer l's are consumed, and
// so on, so a phase finds its weights in LDS. Waves 8-11 issue the copies
// and wait for them by count (vector loads complete in order); waves 0-7
// poll and compute and never issue a copy, so a poll never waits behind
// one. Q4 matrices run as Q8_0 rows of their nibble values (q4_row's chains
// are q8_row's with q = 0..15: the same products in the same order) plus the
// bias term dot_bf16_f32(bias row, block_sums(x)) (scalar.rs:334-359,
// 654-674, 708-740), the block sums formed once per phase.
//
// Attention: keys are cached chain-major per key (the 64 values score lane
// u of 4 multiplies are contiguous), so the score lanes load them straight
// into registers before the q / k / v poll. A context longer than one
// 256-key block (the reference's ATTN_BLOCK) runs block by block, merging
// the partials as scalar.rs attn_merge does, with glibc's expf restated.
//
// Compiled with -ffp-contract=off; __fmaf_rn / __fma_rn exactly where the
// CPU code calls std::fma. What comes from the host: RoPE's cos / sin per
// position (the CPU restatement's own libm calls), sqrt(n_embd), and the
// expf table (2^(i/32), i < 32, rounded to double).

#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "f32_m1.h"
#include "gemma3.h"
#include "nncpu_hip.h"
#include "ops_dev.h"

namespace {

using nnh::F32Mat;
using nnh::lds_barrier;
using nnh::xor_get;

constexpr int ATTN_BLOCK = 256;  // model/mod.rs:84-87
constexpr int E_MAX = 2048;      // residual width
constexpr int PK_NT = 1024;      // threads per workgroup
constexpr int PK_POLL = 512;     // threads 0..511 (waves 0-7) poll
constexpr int PK_LOADERS = 4;    // waves 8-11 copy weights into LDS, on their own schedule
constexpr int PK_CW = PK_POLL;   // threads 0..511 compute (the pollers); waves 12-15 idle in matmul workgroups
constexpr int PK_S = 4;          // attention workgroups per query head
constexpr int PK_KE = E_MAX / PK_POLL;  // residual values per poller thread
constexpr int PK_KF = 16;        // tagged values per poller thread, longest vector (8192)
constexpr int PK_LDS = 156 * 1024;
constexpr long PK_SPIN = 1L << 21;  // poll rounds (each ~1 us) before a wait gives up

// hsum8 of lanes 0..7's values, by lane exchanges (valid at lane 0):
// xor-4 gives v_l + v_{l+4}, xor-1 and xor-2 then add those pairs as hsum8 does.
__device__ __forceinline__ float hsum8_lanes(float a) {
    const float p = __fadd_rn(a, __shfl_xor(a, 4, 64));
    const float q = __fadd_rn(p, __shfl_xor(p, 1, 64));
    return __fadd_rn(q, __shfl_xor(q, 2, 64));
}

}  // namespace

namespace {

// A chain input in LDS, transposed: element e of a dim-vector (dim a
// multiple of 128) at (e % 8) * S + e / 8, S = dim / 8 + 4, so FMA lane l's
// values are contiguous (16-byte reads) and the 4-float pad spreads the eight
// lanes' reads over the banks.
__host__ __device__ __forceinline__ int tstride(int dim) { return dim / 8 + 4; }
__device__ __forceinline__ void tput(float* xt, int S, int e, float v) { xt[(e & 7) * S + (e >> 3)] = v; }

// hsum8 of the eight FMA lanes' sums of squares of a transposed dim-vector
// (dim % 128 == 0), run by lanes 0..7 of the calling wave; valid at lane 0.
// A lane's values are read from LDS 12 float4s at a time, all issued before
// that chunk's FMAs.
__device__ __forceinline__ float chain_sumsq(const float* xt, int dim, int lane) {
    constexpr int CH = 12;
    float a = 0.0f;
    if (lane < 8) {
        const float4* p = (const float4*)(xt + lane * tstride(dim));
        const int n = dim / 32;
        for (int m = 0; m < n; m += CH) {
            float4 b[CH];
#pragma unroll
            for (int k = 0; k < CH; ++k) b[k] = p[min(m + k, n - 1)];  // past the end: a spare read
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                if (m + k < n) {
                    a = __fmaf_rn(b[k].x, b[k].x, a);
                    a = __fmaf_rn(b[k].y, b[k].y, a);
                    a = __fmaf_rn(b[k].z, b[k].z, a);
                    a = __fmaf_rn(b[k].w, b[k].w, a);
                }
            }
        }
    }
    return hsum8_lanes(a);
}


// ---- tagged hand-offs ----------------------------------------------------------------------

__device__ __forceinline__ void tstore(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tload(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int flag_load(const int* p) {
    return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void flag_raise(int* p) {
    __hip_atomic_fetch_or(p, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread t of nt polls values t, t + nt, ... (< n, K per thread) of src
// until each carries `tag`, then stores the floats to dst[i] (LDS). False
// when the wait runs out (the error flag is raised) or another workgroup
// raised it.
template <int K>
__device__ bool poll_tagged(const uint64_t* src, int n, int t, int nt, uint32_t tag, int* err, float* dst) {
    uint64_t w[K];
    for (long r = 0; r < PK_SPIN; ++r) {
#pragma unroll
        for (int k = 0; k < K; ++k) w[k] = tload(src + min(t + nt * k, n - 1));
        bool ok = true;
#pragma unroll
        for (int k = 0; k < K; ++k) ok = ok && (uint32_t)(w[k] >> 32) == tag;
        if (ok) {
#pragma unroll
            for (int k = 0; k < K; ++k)
                if (t + nt * k < n) dst[t + nt * k] = __uint_as_float((uint32_t)w[k]);
            return true;
        }
        if ((r & 63) == 63 && flag_load(err)) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    flag_raise(err);
    return false;
}

// Poller thread t reads values t, t + PK_POLL, ... (< n, K per thread) into
// dst (LDS), waiting for any whose tag is not yet current.
template <int K>
__device__ bool read_tagged(const uint64_t* src, int n, int t, uint32_t tag, int* err, float* dst) {
    uint32_t stale = 0;
#pragma unroll
    for (int k = 0; k < K; ++k)
        if (t + PK_POLL * k < n) stale |= 1u << k;
    for (long r = 0; stale; ++r) {
        // Every stale value re-read at once: one round trip per round.
        uint64_t w[K];
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (stale & (1u << k)) w[k] = tload(src + t + PK_POLL * k);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if ((stale & (1u << k)) && (uint32_t)(w[k] >> 32) == tag) {
                dst[t + PK_POLL * k] = __uint_as_float((uint32_t)w[k]);
                stale &= ~(1u << k);
            }
        }
        if (!stale) break;
        if (r >= PK_SPIN || ((r & 63) == 63 && flag_load(err))) {
            flag_raise(err);
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    return true;
}

constexpr long PK_LSPIN = 1L << 24;  // LDS-wait rounds before a wait gives up

// A barrier of `waves` waves on an LDS counter, for a subset of the
// workgroup (the loader waves never join one). gen: arrivals expected so
// far, kept by the caller.
__device__ __forceinline__ bool lbar(int* ctr, int& gen, int waves) {
    gen += waves;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (long r = 0; r < PK_LSPIN; ++r) {
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= gen) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}
// The poller waves' barrier.
__device__ __forceinline__ bool pbar(int* ctr, int& gen) { return lbar(ctr, gen, PK_POLL / 64); }

// Wait until the LDS counter *p >= v; false on a timeout or an abort.
__device__ __forceinline__ bool lds_wait_ge(int* p, int v, int* abort_flag) {
    for (long r = 0; r < PK_LSPIN; ++r) {
        if (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= v) return true;
        if (__hip_atomic_load(abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

// ---- weight copies into LDS ------------------------------------------------------------

// Producer i of `parts` owns rows [i * total / parts, (i + 1) * total /
// parts) (32-bit: total * parts < 2^31, which nngd_create checks).
__host__ __device__ __forceinline__ int row_first(int total, int parts, int i) {
    return (int)((uint32_t)(i * total) / (uint32_t)parts);
}
__host__ __device__ __forceinline__ void row_range(int total, int parts, int i, int* r0, int* r1) {
    *r0 = row_first(total, parts, i);
    *r1 = row_first(total, parts, i + 1);
}

// A matmul workgroup's rows of each phase's matrices.
struct Rows {
    int q0, q1, o0, o1, f0, f1, d0, d1;
};

// Bytes of a row in the 16-lane layout (Q8 groups of 8 blocks) and of its
// padded scale row.
__host__ __device__ __forceinline__ uint32_t qrow_bytes(const F32Mat& m) { return (uint32_t)((m.nb + 7) / 8) * 256; }
__host__ __device__ __forceinline__ uint32_t srow_bytes(const F32Mat& m) { return (uint32_t)m.nbp * 2; }
// A Q4 bias row: nb BF16 values, zero-padded to whole 16-byte pieces (so a
// copy's last piece never spills into the next run's slots).
__host__ __device__ __forceinline__ uint32_t brow_elems(int nb) { return (uint32_t)((nb + 7) / 8) * 8; }

// Rows [lo, hi) of m into LDS row slots slot0..: v(src, bytes, LDS offset)
// for the quants, then the scales, then (Q4) the bias rows.
template <class V>
__host__ __device__ __forceinline__ void visit_rows(V&& v, const F32Mat& m, int lo, int hi, int slot0, uint32_t wdst,
                                                    uint32_t sdst, uint32_t bdst) {
    if (hi <= lo) return;
    const uint32_t qb = qrow_bytes(m), sb = srow_bytes(m);
    v(m.fq + (size_t)lo * qb, (uint32_t)(hi - lo) * qb, wdst + (uint32_t)slot0 * qb);
    v((const uint8_t*)(m.fs + (size_t)lo * m.nbp), (uint32_t)(hi - lo) * sb, sdst + (uint32_t)slot0 * sb);
    if (m.bi) {
        const uint32_t bb = 2 * brow_elems(m.nb);
        v((const uint8_t*)m.bi + (size_t)lo * bb, (uint32_t)(hi - lo) * bb, bdst + (uint32_t)slot0 * bb);
    }
}

}  // namespace

// LDS byte offsets of a matmul workgroup, and the copy instructions each
// loader wave issues per phase (the most any workgroup needs).
struct PkGeom {
    uint32_t qw, qs, ow, os, fw, fs, dw, ds, qb, ob, fb, db, xs, y, in, xt, res, bc, h, wtab, bytes;
    int kq, ko, kf, kd;
};

struct PkArgs {
    int n_layer, E, F, H, KV, QD, KVD, A, M;
    float eps, attn_scale, embd_scale;
    PkGeom g;
    F32Mat geo[4];              // geometry (no pointers) of q / k / v, o, gate / up, down
    const uint64_t* wptr;       // [n_layer][7] x (quants, scales, Q4 bias rows or 0) of q k v o gate up down
    int q4;                     // the layer matrices are Q4 (bias rows, block sums)
    const float* norms;         // per layer, ns apart: attn, q, k, post_attn, ffn, post_ffw
    size_t ns;
    uint16_t *kc, *vc;          // caches [n_layer][n_ctx][n_kv * HD]: K chain-major per key, V natural
    size_t kv_layer;
    const float *cos_t, *sin_t; // RoPE tables [2][n_ctx][HD / 2]: sliding (local) base, then global
    int n_ctx, window, swa_period;
    const uint64_t* tok;  // the token; the embedding table (the tied lm_head): quants, scales, Q4 biases
    const int8_t* tq;
    const uint16_t* ts;
    const uint16_t* tb;   // null: Q8_0
    const float* out_norm;
    const int *pos_p, *step_p;
    const uint32_t* seq_p;  // steps run on this model so far: the tags' base
    uint64_t *t_qkv, *t_attn, *t_o, *t_h, *t_down;
    float *record, *y;
    size_t rec_stride;
    const uint64_t* expt;  // glibc_expf's table
    int* err;
};

namespace {

// A matmul workgroup's rows (workgroup mw of a.M).
__host__ __device__ inline Rows rows_of(const PkArgs& a, int mw) {
    Rows r;
    row_range(a.QD + 2 * a.KVD, a.M, mw, &r.q0, &r.q1);
    row_range(a.E, a.M, mw, &r.o0, &r.o1);
    row_range(a.F, a.M, mw, &r.f0, &r.f1);
    row_range(a.E, a.M, mw, &r.d0, &r.d1);
    return r;
}

// The contiguous runs of bytes a matmul workgroup (rows rw) copies into LDS
// for a phase of layer Ly, in order: v(src, bytes, LDS offset) for each.
// mat(j): matrix j (q k v o gate up down) of the layer.
template <class Mat, class V>
__host__ __device__ __forceinline__ void visit_phase(const PkArgs& a, Mat&& mat, int phase, const Rows& rw, V&& v) {
    const PkGeom& g = a.g;
    if (phase == 0) {
        const int r0 = rw.q0, r1 = rw.q1, kb = a.QD, vb = a.QD + a.KVD, ve = a.QD + 2 * a.KVD;
        visit_rows(v, mat(0), r0, min(r1, kb), 0, g.qw, g.qs, g.qb);
        visit_rows(v, mat(1), max(r0, kb) - kb, min(r1, vb) - kb, max(r0, kb) - r0, g.qw, g.qs, g.qb);
        visit_rows(v, mat(2), max(r0, vb) - vb, min(r1, ve) - vb, max(r0, vb) - r0, g.qw, g.qs, g.qb);
    } else if (phase == 2) {
        visit_rows(v, mat(3), rw.o0, rw.o1, 0, g.ow, g.os, g.ob);
    } else if (phase == 3) {
        visit_rows(v, mat(4), rw.f0, rw.f1, 0, g.fw, g.fs, g.fb);
        visit_rows(v, mat(5), rw.f0, rw.f1, rw.f1 - rw.f0, g.fw, g.fs, g.fb);
    } else {
        visit_rows(v, mat(6), rw.d0, rw.d1, 0, g.dw, g.ds, g.db);
    }
}

// Which geometry matrix j (q k v o gate up down) has.
__host__ __device__ __forceinline__ int geo_of(int j) { return j < 3 ? 0 : j == 3 ? 1 : j < 6 ? 2 : 3; }

__host__ __device__ __forceinline__ int chunks_of(uint32_t len) { return (int)((len + 1023) >> 10); }

__host__ int phase_chunks(const PkArgs& a, const F32Mat* w7, int phase, int mw) {
    int c = 0;
    visit_phase(a, [&](int j) { return w7[j]; }, phase, rows_of(a, mw), [&](const uint8_t*, uint32_t len, uint32_t) { c += chunks_of(len); });
    return c;
}

// One 16-byte piece global -> LDS (lane l's bytes at LDS address dst + 16 l,
// dst uniform). As asm, so the compiler neither waits for it nor reorders
// LDS reads around it; the waits are explicit.
__device__ __forceinline__ void copy16(const uint8_t* src, uint32_t dst) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(dst) : "memory");
}

// Loader wave lw issues exactly k copy instructions for a phase's runs
// (1 KB chunks lw, lw + PK_LOADERS, ...; past the last chunk it copies the
// last one again, the same bytes to the same place), so every loader wave's
// count per phase is the same known number. Lanes past a run's end are
// masked off.
// The pointers of a layer's matrices from the LDS table (uniform values,
// moved to scalar registers).
__device__ __forceinline__ const void* lds_ptr(const uint64_t* p) {
    const uint64_t v = *p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const void*)(((uint64_t)hi << 32) | lo);
}
struct LdsMats {
    const PkArgs* a;
    const uint64_t* tab;  // this layer's 7 x (quants, scales, bias rows) in LDS
    __device__ __forceinline__ F32Mat operator()(int j) const {
        F32Mat m = a->geo[geo_of(j)];
        m.fq = (const uint8_t*)lds_ptr(tab + 3 * j);
        m.fs = (const uint16_t*)lds_ptr(tab + 3 * j + 1);
        m.bi = a->q4 ? (const uint16_t*)lds_ptr(tab + 3 * j + 2) : nullptr;
        return m;
    }
};

__device__ void issue(const PkArgs& a, const LdsMats& mats, int phase, const Rows& rw, int k, int lw, int lane,
                      uint32_t lds) {
    int total = 0;
    visit_phase(a, mats, phase, rw, [&](const uint8_t*, uint32_t len, uint32_t) { total += chunks_of(len); });
    for (int i = 0; i < k; ++i) {
        const int c = min(lw + PK_LOADERS * i, total - 1);
        const uint8_t* src = nullptr;
        uint32_t len = 0, dst = 0;
        int cs = 0, c0 = 0;
        visit_phase(a, mats, phase, rw, [&](const uint8_t* s_, uint32_t l_, uint32_t d_) {
            if (c >= cs) {  // the last run starting at or before chunk c
                src = s_;
                len = l_;
                dst = d_;
                c0 = cs;
            }
            cs += chunks_of(l_);
        });
        const uint32_t off = (uint32_t)(c - c0) * 1024, o = off + (uint32_t)lane * 16;
        if (o < len) copy16(src + o, lds + dst + off);
    }
}

// ---- the bit-exact row sums, weights in LDS ----------------------------------------------
// gemv_f32_kernel's arithmetic (scalar.rs:626-649): chain j of a row
// (element j of every 32-block) over the blocks in order, acc = fma(f32(q) *
// bf16(s), x, acc), then v[l] = (acc_l + acc_{8+l}) + (acc_{16+l} +
// acc_{24+l}), hsum8. w: the row's 16-lane groups (lane j's 16 bytes of
// group g at g * 256 + 16 j: byte 2i element j of block 8g + i, byte 2i + 1
// element j + 16); s: its BF16 scales; x: the input, natural order.

// One 8-block group of a lane's chains, read from LDS: the 16-byte piece,
// the 8 BF16 scales, and x for chain j (and, 16 lanes per row, j + 16).
template <bool TWO>
struct Grp {
    uint4 q, s;
    float x0[8], x1[TWO ? 8 : 1];
    __device__ __forceinline__ void read(const uint8_t* w, const uint16_t* sc, const float* x, int g, int j) {
        q = *(const uint4*)(w + g * 256 + (TWO ? j : (j & 15)) * 16);
        s = *(const uint4*)(sc + g * 8);
        const float* xb = x + 256 * g + j;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x0[i] = xb[32 * i];
            if (TWO) x1[i] = xb[32 * i + 16];
        }
    }
    // Blocks i < nblk (all 8 when FULL) into the chains; hs: the byte of a
    // pair a one-chain lane takes (0 or 8), applied to the piece once so the
    // per-block byte selects are constants.
    template <bool FULL>
    __device__ __forceinline__ void run(float& a0, float& a1, int nblk, int hs) const {
        uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        const uint32_t sw[4] = {s.x, s.y, s.z, s.w};
        if (!TWO) {
#pragma unroll
            for (int k = 0; k < 4; ++k) qw[k] >>= hs;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (FULL || i < nblk) {
                const float sb = bf16f((sw[i >> 1] >> (16 * (i & 1))) & 0xffffu);
                const uint32_t qq = qw[i >> 1] >> (16 * (i & 1));
                if (TWO) {
                    a0 = __fmaf_rn((float)(int8_t)(qq & 0xffu) * sb, x0[i], a0);
                    a1 = __fmaf_rn((float)(int8_t)((qq >> 8) & 0xffu) * sb, x1[TWO ? i : 0], a1);
                } else {
                    a0 = __fmaf_rn((float)(int8_t)(qq & 0xffu) * sb, x0[i], a0);
                }
            }
        }
    }
};

// The chains of one row over its groups in order, the next group's LDS
// reads issued before the current group's arithmetic.
template <bool TWO>
__device__ __forceinline__ void row_chains(const uint8_t* w, const uint16_t* sc, const float* x, int nb, int j,
                                           float& a0, float& a1) {
    const int ng = nb / 8, hs = TWO ? 0 : 8 * (j >> 4);
    Grp<TWO> A, B;
    int g = 0;
    if (ng > 0) A.read(w, sc, x, 0, j);
    for (; g + 1 < ng; g += 2) {
        B.read(w, sc, x, g + 1, j);
        A.template run<true>(a0, a1, 8, hs);
        if (g + 2 < ng) A.read(w, sc, x, g + 2, j);
        B.template run<true>(a0, a1, 8, hs);
    }
    if (g < ng) A.template run<true>(a0, a1, 8, hs);
    if (nb % 8) {
        B.read(w, sc, x, ng, j);
        B.template run<false>(a0, a1, nb % 8, hs);
    }
}

// 16 lanes per row, lane j (0..15) running chains j and j + 16; the sum is
// valid at j == 0.
__device__ float row16(const uint8_t* w, const uint16_t* s, const float* x, int nb, int j) {
    float a0 = 0.0f, a1 = 0.0f;
    row_chains<true>(w, s, x, nb, j, a0, a1);
    const float u = __fadd_rn(a0, xor_get(a0, 8));
    const float v = __fadd_rn(a1, xor_get(a1, 8));
    const float uv = __fadd_rn(u, v);
    const float p = __fadd_rn(uv, xor_get(uv, 4));
    const float q = __fadd_rn(p, xor_get(p, 1));
    return __fadd_rn(q, xor_get(q, 2));
}

// 32 lanes per row, lane j (0..31) running chain j alone: lanes j and j + 16
// read the same piece and take its even / odd bytes. Valid at j == 0.
__device__ float row32(const uint8_t* w, const uint16_t* s, const float* x, int nb, int j) {
    float a = 0.0f, unused = 0.0f;
    row_chains<false>(w, s, x, nb, j, a, unused);
    const float u = __fadd_rn(a, xor_get(a, 8));
    const float v = __fadd_rn(u, xor_get(u, 16));
    const float p = __fadd_rn(v, xor_get(v, 4));
    const float q = __fadd_rn(p, xor_get(p, 1));
    return __fadd_rn(q, xor_get(q, 2));
}

// The Q4 bias term dot_bf16_f32(bias row, xs) (scalar.rs:334-347): lane l
// of an 8-lane group accumulates elements 8c + l (fused), hsum8 across the
// group, then the tail in order (unfused). b: the row's biases, xs: the
// block sums, both in LDS. Valid at l == 0.
__device__ __forceinline__ float bias_dot(const uint16_t* b, const float* xs, int nb, int l) {
    const int body = nb & ~7;
    float acc = 0.0f;
    for (int c = 0; c < body; c += 8) acc = __fmaf_rn(bf16f(b[c + l]), xs[c + l], acc);
    float s = hsum8_lanes(acc);
    for (int i = body; i < nb; ++i) s = __fadd_rn(s, __fmul_rn(bf16f(b[i]), xs[i]));
    return s;
}

// block_sums (scalar.rs:355-359) of x (LDS) into xs, a thread per block.
__device__ __forceinline__ void block_sums_lds(const float* x, int nb, float* xs, int tid) {
    for (int b = tid; b < nb; b += PK_CW) {
        const float4* c = (const float4*)(x + 32 * b);
        float e[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 f = c[i];
            e[4 * i] = f.x, e[4 * i + 1] = f.y, e[4 * i + 2] = f.z, e[4 * i + 3] = f.w;
        }
        float v[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) v[l] = __fadd_rn(__fadd_rn(__fadd_rn(e[l], e[8 + l]), e[16 + l]), e[24 + l]);
        xs[b] = __fadd_rn(__fadd_rn(__fadd_rn(v[0], v[4]), __fadd_rn(v[1], v[5])),
                          __fadd_rn(__fadd_rn(v[2], v[6]), __fadd_rn(v[3], v[7])));
    }
}

// ---- matmul workgroups -----------------------------------------------------------------

// The pollers' part of P0 / P3, among the poller waves only: x +=
// RMSNorm(in) * g1 (in: the polled vector in LDS, natural order), then y =
// RMSNorm(x) * g2 into Y. Wave 0's lanes 0..7 run the norm chains. g1v /
// g2v: the thread's elements of the gammas, loaded at the start of the pass
// (their loads overlap the wait for the input).
__device__ bool residual_norms(const PkArgs& a, int tid, const float* in, float (&xr)[PK_KE], const float (&g1v)[PK_KE],
                               const float (&g2v)[PK_KE], float* xt, float* Y, float* bc, int* pctr, int& pgen,
                               float* rec, bool add) {
    const int E = a.E, S = tstride(E);
    bool ok = true;
    if (add) {
#pragma unroll
        for (int k = 0; k < PK_KE; ++k) {
            const int i = tid + PK_POLL * k;
            if (i < E) tput(xt, S, i, in[i]);
        }
        ok = pbar(pctr, pgen) && ok;
        if (tid < 64) {
            const float r = chain_sumsq(xt, E, tid);
            if (tid == 0) bc[0] = rms_of(r, E, a.eps);
        }
        ok = pbar(pctr, pgen) && ok;
        const float s1 = bc[0];
#pragma unroll
        for (int k = 0; k < PK_KE; ++k) {
            const int i = tid + PK_POLL * k;
            if (i < E) {
                xr[k] = __fadd_rn(xr[k], __fmul_rn(__fmul_rn(in[i], s1), g1v[k]));
                if (rec) rec[i] = xr[k];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < PK_KE; ++k) {
        const int i = tid + PK_POLL * k;
        if (i < E) tput(xt, S, i, xr[k]);
    }
    ok = pbar(pctr, pgen) && ok;
    if (tid < 64) {
        const float r = chain_sumsq(xt, E, tid);
        if (tid == 0) bc[0] = rms_of(r, E, a.eps);
    }
    ok = pbar(pctr, pgen) && ok;
    const float s2 = bc[0];
#pragma unroll
    for (int k = 0; k < PK_KE; ++k) {
        const int i = tid + PK_POLL * k;
        if (i < E) Y[i] = __fmul_rn(__fmul_rn(xr[k], s2), g2v[k]);
    }
    return ok;
}

// The Q4 block sums of a phase's input are formed by the compute waves
// right before their rows, each wave announcing its share on an LDS counter
// (`bs.ctr`); a row waits for all of them only before its bias term, so the
// row chains run while the other waves finish the sums (no barrier between).
struct BsumWait {
    int* ctr;   // arrivals of the compute waves so far (all passes)
    int want;   // arrivals that complete this pass's sums
    int* abort;
};
__device__ __forceinline__ void bsum_wait(const BsumWait& bs, bool& ready) {
    if (ready) return;
    if (!lds_wait_ge(bs.ctr, bs.want, bs.abort)) *bs.abort = 1;
    ready = true;
}

// A phase's rows (nrows of matrix geometry m, weights w / scales sc / Q4
// bias rows bi (null: Q8_0) in LDS, input x and its block sums xs in LDS),
// NB: the rows' block count when known at compile time. A Q4 row is
// q4_row's sum plus its bias term (gemv_q4_rows: y + bias).
template <int NB>
__device__ __forceinline__ void rows32(const F32Mat& m, const uint8_t* w, const uint8_t* sc, const uint16_t* bi,
                                       const float* xs, const float* x, int nrows, uint64_t* out, uint32_t tag,
                                       int tid, const BsumWait& bs) {
    const int nb = NB ? NB : m.nb;
    const uint32_t qb = NB ? (uint32_t)((NB + 7) / 8) * 256 : qrow_bytes(m), sb = srow_bytes(m);
    bool ready = false;
    for (int slot = tid >> 5; slot < nrows; slot += PK_CW / 32) {
        float v = row32(w + slot * qb, (const uint16_t*)(sc + slot * sb), x, nb, tid & 31);
        if (bi) {
            bsum_wait(bs, ready);
            v = __fadd_rn(v, bias_dot(bi + slot * brow_elems(nb), xs, nb, tid & 7));
        }
        if ((tid & 31) == 0) tstore(out + slot, v, tag);
    }
}
template <int NB>
__device__ __forceinline__ void rows16(const F32Mat& m, const uint8_t* w, const uint8_t* sc, const uint16_t* bi,
                                       const float* xs, const float* x, int nrows, float* res, int tid,
                                       const BsumWait& bs) {
    const int nb = NB ? NB : m.nb;
    const uint32_t qb = NB ? (uint32_t)((NB + 7) / 8) * 256 : qrow_bytes(m), sb = srow_bytes(m);
    bool ready = false;
    for (int slot = tid >> 4; slot < nrows; slot += PK_CW / 16) {
        float v = row16(w + slot * qb, (const uint16_t*)(sc + slot * sb), x, nb, tid & 15);
        if (bi) {
            bsum_wait(bs, ready);
            v = __fadd_rn(v, bias_dot(bi + slot * brow_elems(nb), xs, nb, tid & 7));
        }
        if ((tid & 15) == 0) res[slot] = v;
    }
}

// The matmul workgroups. Waves 8-11 (loaders) copy each layer's rows of
// each matrix into its LDS region as soon as the region's previous layer is
// consumed, wait for the copies and count them landed; they never meet the
// other waves at a barrier, so a slow copy never holds up a phase that does
// not need it. Waves 0-7 poll the inputs, run the norms and compute,
// running the layers as a loop over phases, ph = 0 (q / k / v), 1 (o), 2
// (gate / up), 3 (down), with one copy of each piece of code (the step's
// code stays small enough for the instruction cache). Waves 12-15 have no
// work here. A last pass (mw 0 only) forms the final norm.
template <int NBE, int NBQ, int NBF, bool Q4>
__device__ __forceinline__ void matmul_wg(const PkArgs& a, uint8_t* lds, uint32_t base) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, mw = blockIdx.x - a.A;
    const bool poller = (int)threadIdx.x < PK_POLL;
    const PkGeom& g = a.g;
    const uint32_t lbase = (uint32_t)(uintptr_t)lds;
    float* Y = (float*)(lds + g.y);
    float* XT = (float*)(lds + g.xt);
    float* RES = (float*)(lds + g.res);
    float* BC = (float*)(lds + g.bc);
    int* ABORT = (int*)(BC + 1);
    int* PCTR = (int*)(BC + 2);    // the compute waves' barrier
    int* FREED = (int*)(BC + 4);   // [3] layers consumed of the q / k / v, o, gate / up + down regions
    int* LANDED = (int*)(BC + 8);  // [4] loader-wave copies landed of q / k / v, o, gate / up, down
    int* BSUM = (int*)(BC + 12);   // Q4: compute waves done with the pass's block sums
    float* H = (float*)(lds + g.h);
    float* IN = (float*)(lds + g.in);
    float* XS = (float*)(lds + g.xs);  // Q4: the block sums of the phase's input
    const int E = a.E, L = a.n_layer;
    const Rows rw = rows_of(a, mw);
    const int q0 = rw.q0, q1 = rw.q1, o0 = rw.o0, o1 = rw.o1, f0 = rw.f0, f1 = rw.f1, d0 = rw.d0, d1 = rw.d1;
    const int nf = f1 - f0;
    if (threadIdx.x < 16) ((int*)BC)[threadIdx.x] = 0;
    // The layers' matrix pointers into LDS (scalar loads of a table read
    // once per layer would each wait a memory round trip).
    uint64_t* WT = (uint64_t*)(lds + g.wtab);
    for (int i = threadIdx.x; i < 21 * L; i += PK_NT) WT[i] = a.wptr[i];
    lds_barrier();  // the last barrier of the whole workgroup
    if ((int)threadIdx.x >= PK_CW + 64 * PK_LOADERS) return;
    if ((int)threadIdx.x >= PK_CW) {
        // ---- loader waves
        const int lw = wave - PK_CW / 64;
        for (int l = 0; l < L; ++l) {
            const LdsMats mats{&a, WT + 21 * l};
#pragma unroll 1
            for (int q = 0; q < 4; ++q) {
                // Region free: its previous layer's phase is done.
                if (!lds_wait_ge(FREED + (q == 3 ? 2 : q), l, ABORT)) {
                    flag_raise(a.err);
                    *ABORT = 1;
                    l = L;
                    break;
                }
                issue(a, mats, q == 0 ? 0 : q + 1, rw, q == 0 ? g.kq : q == 1 ? g.ko : q == 2 ? g.kf : g.kd, lw, lane,
                      lbase);
                __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));
                if (lane == 0) __hip_atomic_fetch_add(LANDED + q, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));
        return;
    }
    // ---- compute waves
    int pgen = 0;  // barrier arrivals so far
    float* rec = (mw == 0) ? a.record + (size_t)(*a.step_p) * a.rec_stride : nullptr;
    float xr[PK_KE];
#pragma unroll
    for (int k = 0; k < PK_KE; ++k) xr[k] = 0.0f;
    const int passes = 4 * L + (mw == 0 ? 1 : 0);
    for (int it = 0; it < passes; ++it) {
        const int l = it >> 2, ph = it & 3;
        const bool fin = l == L;  // the final norm
        const int lv = fin ? L - 1 : l;
        const float* nrm = a.norms + a.ns * lv;  // this layer's norms
        const uint32_t tag = base + (uint32_t)l + 1;
        // The thread index through an empty asm: addresses derived from it
        // are recomputed per pass instead of being held in registers.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        // ---- the input, among the poller waves
        if (poller) {
            bool ok = true;
            // The norms' gammas first (attn +0, post_attn +E+2hd, ffn +2E+2hd,
            // post_ffw +3E+2hd): their loads overlap the wait for the input.
            float g1v[PK_KE], g2v[PK_KE];
            const bool norms = ph == 0 || ph == 2;
            if (norms) {
                const int hd2 = 2 * (a.QD / a.H);
                const float* g1 = ph == 2 ? nrm + E + hd2 : a.norms + a.ns * (l - 1) + 3 * E + hd2;  // ph 0: layer l - 1's
                const float* g2 = fin ? a.out_norm : ph == 2 ? nrm + 2 * E + hd2 : nrm;
#pragma unroll
                for (int k = 0; k < PK_KE; ++k) {
                    const int i = tid + PK_POLL * k;
                    g1v[k] = (i < E && it > 0) ? g1[i] : 0.0f;
                    g2v[k] = i < E ? g2[i] : 0.0f;
                }
            }
            if (it == 0) {
                // The token's row times sqrt(n_embd) (kernels/mod.rs:917-954):
                // Q8_0 q * s; Q4 s * q + bias (byte k of a block: elements k,
                // low nibble, and k + 16).
                const size_t t = (size_t)*a.tok;
#pragma unroll
                for (int k = 0; k < PK_KE; ++k) {
                    const int i = tid + PK_POLL * k;
                    if (i < E) {
                        const float vs = __fmul_rn(bf16f(a.ts[t * (E / 32) + i / 32]), a.embd_scale);
                        if (Q4) {
                            const int e = i & 31;
                            const uint8_t byte = ((const uint8_t*)a.tq)[t * (E / 2) + 16 * (i >> 5) + (e & 15)];
                            const float bs = __fmul_rn(bf16f(a.tb[t * (E / 32) + i / 32]), a.embd_scale);
                            xr[k] = __fadd_rn(__fmul_rn(vs, (float)(e < 16 ? (byte & 15) : (byte >> 4))), bs);
                        } else {
                            xr[k] = __fmul_rn((float)a.tq[t * E + i], vs);
                        }
                    }
                }
            } else {
                const uint64_t* src = ph == 0 ? a.t_down : ph == 1 ? a.t_attn : ph == 2 ? a.t_o : a.t_h;
                const int n = ph == 1 ? a.QD : ph == 3 ? a.F : E;
                float* dst = ph == 1 ? Y : ph == 3 ? H : IN;
                if (!read_tagged<PK_KF>(src, n, tid, ph == 0 ? tag - 1 : tag, a.err, dst)) *ABORT = 1;
            }
            if (norms) {
                // x += RMSNorm(in) * g1, y = RMSNorm(x) * g2 (forward.rs:749-803).
                float* r = (rec && ph == 0 && l > 0) ? rec + (size_t)(l - 1) * E : nullptr;
                ok = pbar(PCTR, pgen) && !*ABORT;
                if (ok && !residual_norms(a, tid, IN, xr, g1v, g2v, XT, Y, BC, PCTR, pgen, r, it > 0)) *ABORT = 1;
            }
            // This phase's weights have landed (all four loader waves).
            if (tid == 0 && !fin && !lds_wait_ge(LANDED + ph, PK_LOADERS * (l + 1), ABORT)) {
                flag_raise(a.err);
                *ABORT = 1;
            }
        }
        if (!pbar(PCTR, pgen)) *ABORT = 1;
        if (*ABORT) break;
        if (fin) {
            for (int i = tid; i < E; i += PK_CW) a.y[i] = Y[i];
            break;
        }
        if (Q4) {
            block_sums_lds(ph == 3 ? H : Y, (ph == 1 ? a.QD : ph == 3 ? a.F : E) / 32, XS, tid);
            __builtin_amdgcn_s_waitcnt(NNH_LGKMCNT0);
            if (lane == 0) __hip_atomic_fetch_add(BSUM, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        const BsumWait bs{BSUM, (PK_CW / 64) * (it + 1), ABORT};
        // ---- the rows: 32 lanes per row (one chain each) where there are
        // few rows, 16 lanes (two chains each) for gate / up; one call site
        // per matrix shape, so a known block count unrolls.
        {
            const int nrows = ph == 0 ? q1 - q0 : ph == 1 ? o1 - o0 : ph == 2 ? 2 * nf : d1 - d0;
            const uint16_t* bi = Q4 ? (const uint16_t*)(lds + (ph == 0   ? g.qb
                                                               : ph == 1 ? g.ob
                                                               : ph == 2 ? g.fb
                                                                         : g.db))
                                      : nullptr;
            if (ph == 2)
                rows16<NBE>(a.geo[2], lds + g.fw, lds + g.fs, bi, XS, Y, nrows, RES, tid, bs);
            else if (ph == 0)
                rows32<NBE>(a.geo[0], lds + g.qw, lds + g.qs, bi, XS, Y, nrows, a.t_qkv + q0, tag, tid, bs);
            else if (ph == 1)
                rows32<NBQ>(a.geo[1], lds + g.ow, lds + g.os, bi, XS, Y, nrows, a.t_o + o0, tag, tid, bs);
            else
                rows32<NBF>(a.geo[3], lds + g.dw, lds + g.ds, bi, XS, H, nrows, a.t_down + d0, tag, tid, bs);
        }
        if (!pbar(PCTR, pgen)) *ABORT = 1;
        // The region is free for the next layer's copies (gate / up only
        // after down: the down input H lives there).
        if (tid == 0 && ph != 2)
            __hip_atomic_store(FREED + (ph == 3 ? 2 : ph), l + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (ph == 2 && tid < nf) tstore(a.t_h + f0 + tid, __fmul_rn(gelu_lane(RES[tid]), RES[nf + tid]), tag);
    }
}

// ---- attention workgroups --------------------------------------------------------------

// The first-maximum scan's step (scalar.rs attn_block): b follows a.
__device__ __forceinline__ float first_max(float a, float b) { return a < b ? b : a; }

// Position of element e in a chain-major key row: score lane u = e % 4
// multiplies elements 8c + u (c = 0 .. HD/8 - 1), then 8c + u + 4.
__host__ __device__ __forceinline__ int kperm(int e, int hd) { return (e & 3) * (hd / 4) + ((e >> 2) & 1) * (hd / 8) + (e >> 3); }

template <int HD>
struct AttnLds {
    static constexpr int EW = HD / PK_S, VCH = EW / 8, ST = ATTN_BLOCK / 8 + 4, VS = ATTN_BLOCK + 8, QS = HD / 8 + 4;
    static constexpr int vt = 0;                                      // uint16 [EW][VS]
    static constexpr int pq = ((EW * VS * 2 + 255) / 256) * 256;      // polled q, k, v: float [3][HD]
    static constexpr int qt = pq + 3 * HD * 4;                        // float [8 * tstride(HD)]
    static constexpr int kt = qt + 8 * (HD / 8 + 4) * 4;
    static constexpr int qs = kt + 8 * (HD / 8 + 4) * 4;              // float [HD]
    static constexpr int ks = qs + HD * 4;
    static constexpr int qe = ks + HD * 4;                            // float [8][QS]
    static constexpr int knp = qe + 8 * QS * 4;                       // uint16 [HD], chain-major
    static constexpr int sc = knp + HD * 2;                           // float [ATTN_BLOCK]
    static constexpr int sct = sc + ATTN_BLOCK * 4;                   // float [8][ST]
    static constexpr int red = sct + 8 * ST * 4;                      // float [32]
    static constexpr int bytes = red + 32 * 4;
};

// A key block [k0, k1] (k1 <= pos): the cached keys (positions < pos) into
// registers, chain-major (lane u of key t: 16-byte pieces u * HD/4 ..), and
// this workgroup's slice of the cached values.
template <int HD>
struct KvRegs {
    using Lay = AttnLds<HD>;
    static constexpr int KR = HD / 32;  // 16-byte pieces of a lane's key values
    static constexpr int VL = (ATTN_BLOCK * Lay::VCH + PK_NT - 1) / PK_NT;
    uint4 kr[KR], vr[VL];
    __device__ __forceinline__ void load(const uint16_t* kc, const uint16_t* vc, size_t kv_dim, int kvh, int es, int k0,
                                         int k1, int pos) {
        const int tid = threadIdx.x, t = tid >> 2, u = tid & 3;
        const int last_cached = min(k1, pos - 1);
        if (k0 + t <= last_cached) {
            const uint16_t* p = kc + (size_t)(k0 + t) * kv_dim + kvh * HD + u * (HD / 4);
#pragma unroll
            for (int c = 0; c < KR; ++c) kr[c] = *(const uint4*)(p + 8 * c);
        }
        const int nv = (last_cached - k0 + 1) * Lay::VCH;
        const uint16_t* vb = vc + (size_t)k0 * kv_dim + kvh * HD + es * Lay::EW;
#pragma unroll
        for (int k = 0; k < VL; ++k) {
            const int q = tid + PK_NT * k;
            if (q < nv) vr[k] = *(const uint4*)(vb + (size_t)(q / Lay::VCH) * kv_dim + 8 * (q % Lay::VCH));
        }
    }
};

// One query head, every layer (forward.rs:326-351 and attn_block /
// attn_merge / attn_finish, scalar.rs:444-548): q / k RMSNorm, NeoX RoPE at
// the current position, the K/V append (by the head of each KV group),
// then per key block: scores by 8-lane FMA dots and hsum8 times the scale,
// the first maximum, exp_lane, the 8-lane sum of the weights over whole
// chunks then the tail in order, the V sum as one FMA chain per output
// element over the keys in order; blocks merged in order; / sum.
template <int HD>
__device__ __forceinline__ void attn_wg(const PkArgs& a, uint8_t* lds, uint32_t base) {
    using Lay = AttnLds<HD>;
    constexpr int HALF = HD / 2, CH = HD / 8, EW = Lay::EW, VCH = Lay::VCH, ST = Lay::ST, VS = Lay::VS, QS = Lay::QS;
    constexpr int KR = KvRegs<HD>::KR, VL = KvRegs<HD>::VL;
    uint16_t* vt = (uint16_t*)(lds + Lay::vt);
    float* pq = (float*)(lds + Lay::pq);
    float* qt = (float*)(lds + Lay::qt);
    float* kt = (float*)(lds + Lay::kt);
    float* qs = (float*)(lds + Lay::qs);
    float* ks = (float*)(lds + Lay::ks);
    float* qe = (float*)(lds + Lay::qe);
    uint16_t* knp = (uint16_t*)(lds + Lay::knp);
    float* sc = (float*)(lds + Lay::sc);
    float* sct = (float*)(lds + Lay::sct);
    float* red = (float*)(lds + Lay::red);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x / PK_S, es = blockIdx.x % PK_S, group = a.H / a.KV, kvh = h / group;
    const size_t kv_dim = (size_t)a.KVD;
    const int pos = *a.pos_p;
    for (int l = 0; l < a.n_layer; ++l) {
        const uint32_t tag = base + (uint32_t)l + 1;
        const bool sliding = a.swa_period > 0 && (l + 1) % a.swa_period != 0;  // load.rs:1156-1160
        const int window = sliding ? a.window : 0;
        uint16_t* kc = a.kc + a.kv_layer * l;
        uint16_t* vc = a.vc + a.kv_layer * l;
        const float* q_norm = a.norms + a.ns * l + a.E;
        const float* k_norm = q_norm + HD;
        const size_t tab = sliding ? 0 : (size_t)a.n_ctx * HALF;
        const int first = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
        const int bf = first / ATTN_BLOCK, bl = pos / ATTN_BLOCK;
        KvRegs<HD> kv;
        {
            const int k0 = max(first, bf * ATTN_BLOCK), k1 = min(pos, bf * ATTN_BLOCK + ATTN_BLOCK - 1);
            kv.load(kc, vc, kv_dim, kvh, es, k0, k1, pos);
        }
        // The norm gammas and RoPE's cos / sin, loaded before the wait.
        const int e = tid < HD ? tid : HD - 1, jr = e % HALF;
        const float qg = q_norm[e], kg = k_norm[e];
        const float cs = a.cos_t[tab + (size_t)pos * HALF + jr], sn = a.sin_t[tab + (size_t)pos * HALF + jr];
        // q of head h, k and v of its KV head.
        if (tid == 0) red[30] = 0.0f;
        lds_barrier();
        if (tid < 3 * HD) {
            const int part = tid / HD, e = tid % HD;
            const int src = part == 0 ? h * HD + e : a.QD + (part - 1) * a.KVD + kvh * HD + e;
            if (!poll_tagged<1>(a.t_qkv + src, 1, 0, 1, tag, a.err, pq + tid)) red[30] = 1.0f;
        }
        lds_barrier();
        if (red[30] != 0.0f) break;
        // q and k RMSNorm: wave 0 runs q's chain, wave 1 k's (transposed copies).
        if (tid < HD) {
            tput(qt, tstride(HD), tid, pq[tid]);
            tput(kt, tstride(HD), tid, pq[HD + tid]);
        }
        lds_barrier();
        if (wave < 2) {
            const float ss = chain_sumsq(wave == 0 ? qt : kt, HD, lane);
            if (lane == 0) red[wave] = rms_of(ss, HD, a.eps);
        }
        lds_barrier();
        if (tid < HD) {
            qs[tid] = __fmul_rn(__fmul_rn(pq[tid], red[0]), qg);
            ks[tid] = __fmul_rn(__fmul_rn(pq[HD + tid], red[1]), kg);
        }
        lds_barrier();
        // RoPE: threads 0..HALF-1 rotate q's pairs (j, j + HALF), HALF..HD-1 k's.
        if (tid < HD) {
            const int j = jr;
            const float* src = tid < HALF ? qs : ks;
            const float x0 = src[j], x1 = src[j + HALF];
            const float r0 = __fsub_rn(__fmul_rn(cs, x0), __fmul_rn(sn, x1));
            const float r1 = __fadd_rn(__fmul_rn(sn, x0), __fmul_rn(cs, x1));
            if (tid < HALF) {
                qe[(j & 7) * QS + (j >> 3)] = r0;
                qe[((j + HALF) & 7) * QS + ((j + HALF) >> 3)] = r1;
            } else {
                knp[kperm(j, HD)] = to_bf16(r0);
                knp[kperm(j + HALF, HD)] = to_bf16(r1);
            }
        }
        lds_barrier();
        // The K/V append (forward.rs:326-351): the head of each KV group.
        if (h % group == 0) {
            if (es == 0 && tid < HD) kc[(size_t)pos * kv_dim + kvh * HD + tid] = knp[tid];
            if (tid < EW)
                vc[(size_t)pos * kv_dim + kvh * HD + es * EW + tid] = to_bf16(pq[2 * HD + es * EW + tid]);
        }
        float acc_o = 0.0f, acc_m = 0.0f, acc_l = 0.0f;
        for (int b = bf; b <= bl; ++b) {
            const int k0 = max(first, b * ATTN_BLOCK), k1 = min(pos, b * ATTN_BLOCK + ATTN_BLOCK - 1);
            const int n = k1 - k0 + 1;
            if (b > bf) kv.load(kc, vc, kv_dim, kvh, es, k0, k1, pos);
            // This slice of the values, transposed into LDS (the new one from q/k/v).
            {
                const int nv = (min(k1, pos - 1) - k0 + 1) * VCH;
#pragma unroll
                for (int k = 0; k < VL; ++k) {
                    const int q = tid + PK_NT * k;
                    if (q < nv) {
                        const int t = q / VCH, e0 = 8 * (q % VCH);
                        const uint32_t w[4] = {kv.vr[k].x, kv.vr[k].y, kv.vr[k].z, kv.vr[k].w};
#pragma unroll
                        for (int i = 0; i < 8; ++i) vt[(e0 + i) * VS + t] = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
                    }
                }
                if (k1 == pos && tid < EW) vt[tid * VS + (pos - k0)] = to_bf16(pq[2 * HD + es * EW + tid]);
            }
            // Scores: four lanes per key (key tid / 4), lane u running the
            // dot's chains u and u + 4 (elements 8c + u and 8c + u + 4, c in
            // order), then (a_u + a_{u+4}), xor-1, xor-2: hsum8's additions
            // in its order.
            {
                const int t = tid >> 2, u = tid & 3;
                float a0 = 0.0f, a1 = 0.0f;
                if (t < n) {
                    uint4* kk = kv.kr;
                    if (k0 + t == pos) {  // the new key, from LDS
#pragma unroll
                        for (int c = 0; c < KR; ++c) kk[c] = *(const uint4*)(knp + u * (HD / 4) + 8 * c);
                    }
                    const float* q0 = qe + u * QS;
                    const float* q1 = qe + (u + 4) * QS;
#pragma unroll
                    for (int c = 0; c < CH; ++c) {
                        const uint4 lo = kk[c / 8], hi = kk[KR / 2 + c / 8];
                        const uint32_t wl[4] = {lo.x, lo.y, lo.z, lo.w}, wh[4] = {hi.x, hi.y, hi.z, hi.w};
                        const int i = c % 8;
                        a0 = __fmaf_rn(q0[c], bf16f((wl[i >> 1] >> (16 * (i & 1))) & 0xffffu), a0);
                        a1 = __fmaf_rn(q1[c], bf16f((wh[i >> 1] >> (16 * (i & 1))) & 0xffffu), a1);
                    }
                }
                float p = __fadd_rn(a0, a1);
                p = __fadd_rn(p, __shfl_xor(p, 1, 64));
                p = __fadd_rn(p, __shfl_xor(p, 2, 64));
                if (t < n && u == 0) sc[t] = __fmul_rn(p, a.attn_scale);
            }
            lds_barrier();
            const float s_t = tid < n ? sc[tid] : -INFINITY;
            // The first maximum over keys in order: a leftmost-maximum tree,
            // with a NaN after key 0 never taken (as the scan's comparison
            // never takes one) and a NaN at key 0 kept (it is never replaced).
            float mv = (tid > 0 && s_t != s_t) ? -INFINITY : s_t;
#pragma unroll
            for (int k = 1; k < 64; k <<= 1) {
                const float o = __shfl_xor(mv, k, 64);
                mv = (lane & k) ? first_max(o, mv) : first_max(mv, o);
            }
            if (lane == 0) red[2 + wave] = mv;
            lds_barrier();
            float m = red[2];
#pragma unroll
            for (int w = 1; w < PK_NT / 64; ++w) m = first_max(m, red[2 + w]);
            if (tid < n) {
                const float pw = exp_lane(__fsub_rn(s_t, m));
                sc[tid] = pw;
                sct[(tid & 7) * ST + (tid >> 3)] = pw;
            }
            lds_barrier();
            if (tid < 64) {
                // The eight add lanes over the whole chunks of 8, in order.
                const int body = n & ~7, K = body / 8;
                float acc = 0.0f;
                if (tid < 8) {
                    const float* p = sct + tid * ST;
                    int k = 0;
                    for (; k + 4 <= K; k += 4) {
                        const float4 v = *(const float4*)(p + k);
                        acc = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(acc, v.x), v.y), v.z), v.w);
                    }
                    for (; k < K; ++k) acc = __fadd_rn(acc, p[k]);
                }
                float ls = hsum8_lanes(acc);
                if (tid == 0) {
                    for (int j = body; j < n; ++j) ls = __fadd_rn(ls, sc[j]);
                    red[2 + PK_NT / 64] = ls;
                }
            }
            lds_barrier();
            const float lsum = red[2 + PK_NT / 64];
            float o = 0.0f;
            if (tid < EW) {
                // V: one FMA chain per element over the keys in order, 8 keys
                // per 16-byte read of the transposed values.
                const uint16_t* vrow = vt + tid * VS;
                const int nbat = (n + 7) / 8;
                for (int bb = 0; bb < nbat; ++bb) {
                    const uint4 v = *(const uint4*)(vrow + 8 * bb);
                    const float4 p0 = *(const float4*)(sc + 8 * bb), p1 = *(const float4*)(sc + 8 * bb + 4);
                    const float vv[8] = {bf16f(v.x & 0xffffu), bf16f(v.x >> 16), bf16f(v.y & 0xffffu), bf16f(v.y >> 16),
                                         bf16f(v.z & 0xffffu), bf16f(v.z >> 16), bf16f(v.w & 0xffffu), bf16f(v.w >> 16)};
                    const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int t = 8 * bb + j;
                        if (t < n) o = t == 0 ? __fmul_rn(pp[j], vv[j]) : __fmaf_rn(pp[j], vv[j], o);
                    }
                }
            }
            if (b == bf) {
                acc_o = o;
                acc_m = m;
                acc_l = lsum;
            } else {
                // scalar.rs:521-537 (gemma3.cpp attn_merge).
                const float mm = acc_m < m ? m : acc_m;
                const float ca = glibc_expf(__fsub_rn(acc_m, mm), a.expt), cb = glibc_expf(__fsub_rn(m, mm), a.expt);
                acc_o = __fmaf_rn(o, cb, __fmul_rn(acc_o, ca));
                acc_m = mm;
                acc_l = __fadd_rn(__fmul_rn(acc_l, ca), __fmul_rn(lsum, cb));
            }
            lds_barrier();  // sc, vt and red are rewritten by the next block
        }
        if (tid < EW) {
            const float inv = acc_l > 0.0f ? __fdiv_rn(1.0f, acc_l) : 0.0f;
            tstore(a.t_attn + h * HD + es * EW + tid, __fmul_rn(acc_o, inv), tag);
        }

    }
}

// The arguments live in device memory (a by-value struct whose address the
// workgroup code takes would be copied to the stack).
// NBE, NBQ, NBF: the block counts of the n_embd-, q-dim- and n_ff-column
// matrices when compiled for them (Gemma-3-1B's), else 0.
template <int HD, int NBE, int NBQ, int NBF, bool Q4>
__global__ __launch_bounds__(PK_NT) void step_kernel(const PkArgs* __restrict__ ap) {
    __shared__ __attribute__((aligned(256))) uint8_t lds[PK_LDS];
    const PkArgs& a = *ap;
    const uint32_t base = *a.seq_p * (uint32_t)a.n_layer;
    if ((int)blockIdx.x < a.A)
        attn_wg<HD>(a, lds, base);
    else
        matmul_wg<NBE, NBQ, NBF, Q4>(a, lds, base);
}

// End of a step: the greedy token is recorded, the position advances.
__global__ void step_end_kernel(const uint64_t* tok, int* tokens_out, int* pos_p, int* step_p, uint32_t* seq_p) {
    tokens_out[*step_p] = (int)*tok;
    *pos_p += 1;
    *step_p += 1;
    *seq_p += 1;
}

// The CPU harness's K cache (natural order) into the chain-major layout.
__global__ void kperm_kernel(const uint16_t* src, uint16_t* dst, size_t rows, int hd) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * hd) return;
    const size_t r = i / hd;
    const int e = (int)(i % hd);
    dst[r * hd + kperm(e, hd)] = src[i];
}

}  // namespace

#define GD_HIP(expr)                                                    \
    do {                                                                \
        hipError_t e_ = (expr);                                         \
        if (e_ != hipSuccess) {                                         \
            m->err = std::string(#expr) + ": " + hipGetErrorString(e_); \
            return 1;                                                   \
        }                                                               \
    } while (0)

extern "C" {

struct nngd_model {
    nng_config c;
    std::vector<nnh_weight*> w;  // 7 * n_layer + 1, lm_head (the tied token_embd) last
    PkArgs args{};
    PkArgs* args_dev = nullptr;
    uint64_t* wptr = nullptr;
    float* norms = nullptr;  // device copy, layout of nng_create
    uint16_t *kc = nullptr, *vc = nullptr, *kstage = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;  // [2][n_ctx][hd/2]: sliding (local) base, then global
    uint64_t* tagged = nullptr;
    float *y = nullptr, *logits = nullptr, *record = nullptr;
    uint64_t* expt = nullptr;
    void* work = nullptr;
    uint64_t* tok = nullptr;
    int *pos = nullptr, *step = nullptr, *tokens = nullptr, *errf = nullptr;
    uint32_t* seq = nullptr;
    uint16_t* bias = nullptr;           // Q4: every layer matrix's bias rows, padded
    std::vector<nnh_weight*> shadow;    // Q4: Q8_0 copies of the layer matrices' nibble values
    int n_gen_max = 0, grid = 0;
    const void* kernel = nullptr;  // the step kernel instance for this model's shapes
    hipStream_t st = nullptr;
    hipGraphExec_t exec = nullptr;
    std::string err;
};

static size_t norm_stride(const nng_config& c) { return 4 * (size_t)c.n_embd + 2 * (size_t)c.head_dim; }

const char* nngd_error(nngd_model* m) { return m->err.c_str(); }

void nngd_free(nngd_model* m) {
    if (!m) return;
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    void* bufs[] = {m->args_dev, m->wptr, m->norms, m->kc,   m->vc,  m->kstage, m->cos_t, m->sin_t, m->tagged, m->y,
                    m->logits, m->record, m->expt, m->work, m->tok,    m->pos,   m->step,  m->tokens, m->errf,
                    m->seq};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (m->bias) (void)hipFree(m->bias);
    for (nnh_weight* w : m->shadow) nnh_free(w);
    if (m->st) (void)hipStreamDestroy(m->st);
    delete m;
}


// glibc_expf on the host (the function the device runs), for the CPU test
// against the platform's expf.
void nngd_expf_batch(const float* x, float* y, size_t n) {
    uint64_t T[32];
    expf_table(T);
    for (size_t i = 0; i < n; ++i) y[i] = glibc_expf(x[i], T);
}

// RoPE tables exactly as gemma3.cpp's rope_neox forms them: ratio =
// pow(base, -2 / n_rot) and inv *= ratio in f32, theta = pos * inv.
static void rope_table(float base, int n_ctx, int hd, float* cs, float* sn) {
    const int half = hd / 2;
    const float ratio = std::pow(base, -2.0f / (float)hd);
    for (int p = 0; p < n_ctx; ++p) {
        float inv = 1.0f;
        for (int i = 0; i < half; ++i) {
            const float theta = (float)p * inv;
            cs[(size_t)p * half + i] = std::cos(theta);
            sn[(size_t)p * half + i] = std::sin(theta);
            inv *= ratio;
        }
    }
}

static uint32_t align256(size_t v) { return (uint32_t)((v + 255) & ~(size_t)255); }

int nngd_create(const nng_config* cfg, const float* norms, nnh_weight* const* weights, int n_weights, int n_gen_max,
                nngd_model** out) {
    nngd_model* m = new nngd_model();
    *out = m;
    m->c = *cfg;
    const nng_config& c = m->c;
    if (n_weights != 7 * c.n_layer + 1 || c.n_head % c.n_kv != 0) {
        m->err = "bad weight count or head grouping";
        return 1;
    }
    if (c.arch != NNG_GEMMA3 || c.rope_mode != NNG_ROPE_NEOX) {
        m->err = "the device decode step runs Gemma-3 (NeoX RoPE); other architectures take nngl_forward";
        return 1;
    }
    if (c.n_embd % 128 || c.n_embd > E_MAX || (c.head_dim != 128 && c.head_dim != 256) || c.n_ff % 32 ||
        c.n_ff > PK_POLL * PK_KF) {
        m->err = "the device step needs n_embd a multiple of 128 up to 2048, head_dim 128 or 256, n_ff up to 8192";
        return 1;
    }
    m->w.assign(weights, weights + n_weights);
    // Layer matrices: Q8_0 as uploaded; Q4 as a Q8_0 copy of the nibble
    // values (the same chains: f32(q) * s with q = 0..15) through the
    // library, whose f32 layout the step reads, plus the bias rows, each
    // zero-padded to whole 16-byte pieces.
    std::vector<F32Mat> f;
    std::vector<uint16_t> bias_host;
    std::vector<size_t> bias_at;
    int wdt = 0;
    for (int i = 0; i < 7 * c.n_layer; ++i) {
        int dt = 0;
        size_t rows = 0, cols = 0;
        if (nnh_weight_info(weights[i], &dt, &rows, &cols)) {
            m->err = std::string("weight info: ") + nnh_last_error();
            return 1;
        }
        if ((dt != NNH_Q8_0 && dt != NNH_Q4S) || (i > 0 && dt != wdt)) {
            m->err = "the device step takes layer matrices all Q8_0 or all Q4";
            return 1;
        }
        wdt = dt;
        const nnh_weight* src = weights[i];
        if (dt == NNH_Q4S) {
            const size_t n = rows * cols, nb = cols / 32, be = brow_elems((int)nb);
            std::vector<uint8_t> raw(n / 2 + n / 8);
            std::vector<int8_t> q8(n);
            nnh_weight* sh = nullptr;
            if (nnh_weight_download(weights[i], raw.data(), raw.size())) {
                m->err = std::string("Q4 download: ") + nnh_last_error();
                return 1;
            }
            for (size_t r = 0; r < rows; ++r)
                for (size_t b = 0; b < nb; ++b)
                    for (int k = 0; k < 16; ++k) {
                        const uint8_t byte = raw[r * cols / 2 + 16 * b + k];
                        q8[r * cols + 32 * b + k] = (int8_t)(byte & 15);
                        q8[r * cols + 32 * b + k + 16] = (int8_t)(byte >> 4);
                    }
            const uint16_t* sc = (const uint16_t*)(raw.data() + n / 2);
            const uint16_t* bi = sc + n / 32;
            if (nnh_upload_q8_0(q8.data(), sc, rows, cols, &sh)) {
                m->err = std::string("Q4 rows as Q8_0: ") + nnh_last_error();
                return 1;
            }
            m->shadow.push_back(sh);
            src = sh;
            bias_at.push_back(bias_host.size());
            for (size_t r = 0; r < rows; ++r) {
                bias_host.insert(bias_host.end(), bi + r * nb, bi + (r + 1) * nb);
                bias_host.insert(bias_host.end(), be - nb, (uint16_t)0);
            }
        }
        nnh_f32_layout l;
        if (nnh_weight_f32_layout(src, &l)) {
            m->err = std::string("weight layout: ") + nnh_last_error();
            return 1;
        }
        f.push_back(F32Mat{(const uint8_t*)l.quants, l.scales, nullptr, (int)l.rows, (int)l.nb, (int)l.nbp});
    }
    if (wdt == NNH_Q4S) {
        GD_HIP(hipMalloc((void**)&m->bias, bias_host.size() * 2));
        GD_HIP(hipMemcpy(m->bias, bias_host.data(), bias_host.size() * 2, hipMemcpyHostToDevice));
        for (int i = 0; i < 7 * c.n_layer; ++i) f[i].bi = m->bias + bias_at[i];
    }
    // The lm_head's layouts too, before any step is captured.
    if (nnh_weight_prepare(m->w.back(), NNH_ACT_F32, 1)) {
        m->err = std::string("lm_head layout: ") + nnh_last_error();
        return 1;
    }
    int dev = 0, cus = 0;
    GD_HIP(hipGetDevice(&dev));
    GD_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int E = c.n_embd, hd = c.head_dim, QD = c.n_head * hd, KVD = c.n_kv * hd, F = c.n_ff;
    PkArgs& a = m->args;
    a.n_layer = c.n_layer;
    a.E = E;
    a.F = F;
    a.H = c.n_head;
    a.KV = c.n_kv;
    a.QD = QD;
    a.KVD = KVD;
    a.A = c.n_head * PK_S;
    a.M = cus - a.A;
    a.eps = c.rms_eps;
    a.attn_scale = c.attn_scale;
    a.embd_scale = std::sqrt((float)E);
    if (a.M < 1 || QD + 2 * KVD < a.M || E < a.M || F < a.M || (long)(QD + 2 * KVD + F) * cus >= (1L << 31)) {
        m->err = "the device step needs every matmul workgroup to own rows of every matrix";
        return 1;
    }
    // LDS of a matmul workgroup: the largest share of each phase's rows.
    auto most = [&](int total) { return (total + a.M - 1) / a.M; };
    const F32Mat &mq = f[0], &mo = f[3], &mf = f[4], &md = f[6];
    PkGeom& g = a.g;
    size_t o = 0;
    g.qw = (uint32_t)o, o = align256(o + (size_t)most(QD + 2 * KVD) * qrow_bytes(mq));
    g.qs = (uint32_t)o, o = align256(o + (size_t)most(QD + 2 * KVD) * srow_bytes(mq));
    g.ow = (uint32_t)o, o = align256(o + (size_t)most(E) * qrow_bytes(mo));
    g.os = (uint32_t)o, o = align256(o + (size_t)most(E) * srow_bytes(mo));
    g.fw = (uint32_t)o;
    const size_t fw_bytes = (size_t)2 * most(F) * qrow_bytes(mf);
    o = align256(o + std::max(fw_bytes, (size_t)F * 4));  // H (the down input) aliases the FFN weights
    g.h = g.fw;
    g.fs = (uint32_t)o, o = align256(o + (size_t)2 * most(F) * srow_bytes(mf));
    g.dw = (uint32_t)o, o = align256(o + (size_t)most(E) * qrow_bytes(md));
    g.ds = (uint32_t)o, o = align256(o + (size_t)most(E) * srow_bytes(md));
    const bool q4 = wdt == NNH_Q4S;
    auto bbytes = [&](int rows, const F32Mat& mm) { return q4 ? (size_t)rows * 2 * brow_elems(mm.nb) : 0; };
    g.qb = (uint32_t)o, o = align256(o + bbytes(most(QD + 2 * KVD), mq));
    g.ob = (uint32_t)o, o = align256(o + bbytes(most(E), mo));
    g.fb = (uint32_t)o, o = align256(o + bbytes(2 * most(F), mf));
    g.db = (uint32_t)o, o = align256(o + bbytes(most(E), md));
    g.y = (uint32_t)o, o = align256(o + (size_t)std::max(E, QD) * 4);
    // The Q4 block sums alias the polled input: formed after the norms have
    // read it, dead before the next phase polls into it.
    g.in = (uint32_t)o, o = align256(o + std::max((size_t)E * 4, q4 ? (size_t)std::max(std::max(E, QD), F) / 32 * 4 : 0));
    g.xs = g.in;
    g.xt = (uint32_t)o, o = align256(o + (size_t)8 * tstride(E) * 4);
    g.res = (uint32_t)o, o = align256(o + (size_t)2 * most(F) * 4);
    g.bc = (uint32_t)o, o = align256(o + 64);
    g.wtab = (uint32_t)o, o = align256(o + (size_t)21 * c.n_layer * 8);
    g.bytes = (uint32_t)o;
    if (o > (size_t)PK_LDS || (hd == 256 ? AttnLds<256>::bytes : AttnLds<128>::bytes) > PK_LDS) {
        m->err = "the device step's LDS share exceeds the workgroup's LDS";
        return 1;
    }
    // The layer table.
    const size_t nn = norm_stride(c) * c.n_layer + E, half = hd / 2;
    GD_HIP(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
    GD_HIP(hipMalloc((void**)&m->norms, nn * 4));
    GD_HIP(hipMemcpy(m->norms, norms, nn * 4, hipMemcpyHostToDevice));
    GD_HIP(hipMalloc((void**)&m->kc, (size_t)c.n_layer * c.n_ctx * KVD * 2));
    GD_HIP(hipMalloc((void**)&m->vc, (size_t)c.n_layer * c.n_ctx * KVD * 2));
    GD_HIP(hipMalloc((void**)&m->kstage, (size_t)c.n_layer * c.n_ctx * KVD * 2));
    std::vector<float> cs(2 * (size_t)c.n_ctx * half), sn(2 * (size_t)c.n_ctx * half);
    rope_table(c.rope_base_swa, c.n_ctx, hd, cs.data(), sn.data());
    rope_table(c.rope_base, c.n_ctx, hd, cs.data() + (size_t)c.n_ctx * half, sn.data() + (size_t)c.n_ctx * half);
    GD_HIP(hipMalloc((void**)&m->cos_t, cs.size() * 4));
    GD_HIP(hipMalloc((void**)&m->sin_t, sn.size() * 4));
    GD_HIP(hipMemcpy(m->cos_t, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->sin_t, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    const size_t ns = norm_stride(c);
    a.geo[0] = f[0], a.geo[1] = f[3], a.geo[2] = f[4], a.geo[3] = f[6];
    a.q4 = q4 ? 1 : 0;
    for (F32Mat& gm : a.geo) gm.fq = nullptr, gm.fs = nullptr, gm.bi = nullptr;
    for (int li = 0; li < c.n_layer; ++li)
        for (int j = 0; j < 7; ++j) {
            const F32Mat& w = f[7 * li + j], &gw = a.geo[geo_of(j)];
            if (w.nb != gw.nb || w.nbp != gw.nbp) {
                m->err = "every layer's matrices must share the first layer's column counts";
                return 1;
            }
        }
    std::vector<uint64_t> wp(21 * (size_t)c.n_layer);
    for (int li = 0; li < c.n_layer; ++li)
        for (int j = 0; j < 7; ++j) {
            wp[21 * li + 3 * j] = (uint64_t)(uintptr_t)f[7 * li + j].fq;
            wp[21 * li + 3 * j + 1] = (uint64_t)(uintptr_t)f[7 * li + j].fs;
            wp[21 * li + 3 * j + 2] = (uint64_t)(uintptr_t)f[7 * li + j].bi;
        }
    GD_HIP(hipMalloc((void**)&m->wptr, wp.size() * 8));
    GD_HIP(hipMemcpy(m->wptr, wp.data(), wp.size() * 8, hipMemcpyHostToDevice));
    a.wptr = m->wptr;
    a.norms = m->norms;
    a.ns = ns;
    a.kc = m->kc;
    a.vc = m->vc;
    a.kv_layer = (size_t)c.n_ctx * KVD;
    a.cos_t = m->cos_t;
    a.sin_t = m->sin_t;
    a.n_ctx = c.n_ctx;
    a.window = c.window;
    a.swa_period = c.swa_period;
    // Copy counts per loader wave: the most chunks any workgroup copies.
    int kmax[5] = {0, 0, 0, 0, 0};
    for (int li = 0; li < c.n_layer; ++li)
        for (int mw = 0; mw < a.M; ++mw)
            for (int ph : {0, 2, 3, 4}) {
                const int ch = phase_chunks(a, f.data() + 7 * li, ph, mw);
                kmax[ph] = std::max(kmax[ph], (ch + PK_LOADERS - 1) / PK_LOADERS);
            }
    g.kq = kmax[0], g.ko = kmax[2], g.kf = kmax[3], g.kd = kmax[4];
    if (g.kq + g.ko + g.kf + g.kd > 63) {
        m->err = "the device step's weight copies exceed the load counter";
        return 1;
    }
    // Tagged hand-off buffers, zero (tag 0 is never current).
    const size_t nt = (size_t)(QD + 2 * KVD) + QD + E + F + E;
    GD_HIP(hipMalloc((void**)&m->tagged, nt * 8));
    GD_HIP(hipMemset(m->tagged, 0, nt * 8));
    a.t_qkv = m->tagged;
    a.t_attn = a.t_qkv + QD + 2 * KVD;
    a.t_o = a.t_attn + QD;
    a.t_h = a.t_o + E;
    a.t_down = a.t_h + F;
    // glibc_expf's table.
    uint64_t T[32];
    expf_table(T);
    GD_HIP(hipMalloc((void**)&m->expt, sizeof T));
    GD_HIP(hipMemcpy(m->expt, T, sizeof T, hipMemcpyHostToDevice));
    m->n_gen_max = n_gen_max;
    GD_HIP(hipMalloc((void**)&m->y, (size_t)E * 4));
    GD_HIP(hipMalloc((void**)&m->logits, (size_t)c.n_vocab * 4));
    GD_HIP(hipMalloc((void**)&m->record, (size_t)std::max(n_gen_max, 1) * c.n_layer * E * 4));
    GD_HIP(hipMalloc(&m->work, nnh_model_argmax_work_bytes(m->w.back())));
    GD_HIP(hipMalloc((void**)&m->tok, 8));
    GD_HIP(hipMalloc((void**)&m->pos, 4));
    GD_HIP(hipMalloc((void**)&m->step, 4));
    GD_HIP(hipMalloc((void**)&m->seq, 4));
    GD_HIP(hipMalloc((void**)&m->errf, 4));
    GD_HIP(hipMemset(m->seq, 0, 4));
    GD_HIP(hipMemset(m->errf, 0, 4));
    GD_HIP(hipMalloc((void**)&m->tokens, (size_t)std::max(n_gen_max, 1) * 4));
    const uint8_t* te = (const uint8_t*)nnh_weight_device_data(m->w.back());
    int edt = 0;
    size_t er = 0, ec = 0;
    if (nnh_weight_info(m->w.back(), &edt, &er, &ec) || er != (size_t)c.n_vocab || ec != (size_t)E ||
        edt != wdt) {
        m->err = "the embedding table must be n_vocab x n_embd, in the layer matrices' format";
        return 1;
    }
    const size_t tn = (size_t)c.n_vocab * E;
    a.tok = m->tok;
    a.tq = (const int8_t*)te;
    a.ts = (const uint16_t*)(te + (edt == NNH_Q4S ? tn / 2 : tn));
    a.tb = edt == NNH_Q4S ? (const uint16_t*)(te + tn / 2 + tn / 16) : nullptr;
    a.out_norm = m->norms + ns * c.n_layer;
    a.pos_p = m->pos;
    a.step_p = m->step;
    a.seq_p = m->seq;
    a.record = m->record;
    a.y = m->y;
    a.rec_stride = (size_t)c.n_layer * E;
    a.expt = m->expt;
    a.err = m->errf;
    m->grid = a.A + a.M;
    GD_HIP(hipMalloc((void**)&m->args_dev, sizeof(PkArgs)));
    GD_HIP(hipMemcpy(m->args_dev, &a, sizeof(PkArgs), hipMemcpyHostToDevice));
    // Gemma-3-1B's shapes have an instance of their own (its row loops
    // unroll); Q4 layer matrices one of their own (the bias term).
    const bool g1b = hd == 256 && E == 1152 && QD == 1024 && F == 6912;
    if (q4)
        m->kernel = g1b ? (const void*)step_kernel<256, 36, 32, 216, true>
                        : hd == 256 ? (const void*)step_kernel<256, 0, 0, 0, true>
                                    : (const void*)step_kernel<128, 0, 0, 0, true>;
    else
        m->kernel = g1b ? (const void*)step_kernel<256, 36, 32, 216, false>
                        : hd == 256 ? (const void*)step_kernel<256, 0, 0, 0, false>
                                    : (const void*)step_kernel<128, 0, 0, 0, false>;
    // Every workgroup must be resident at once.
    int per_cu = 0;
    GD_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, m->kernel, PK_NT, 0));
    if (per_cu < 1) {
        m->err = "the device step kernel does not fit a CU";
        return 1;
    }
    return 0;
}

// Queue one decode step on m->st (eagerly, or into a graph being captured).
static int queue_step(nngd_model* m) {
    void* args[] = {&m->args_dev};
    GD_HIP(hipLaunchCooperativeKernel(m->kernel, dim3(m->grid), dim3(PK_NT), args, 0, m->st));
    if (nnh_model_argmax_dev(m->w.back(), m->y, m->logits, m->work, m->tok, m->st)) {
        m->err = std::string("lm_head: ") + nnh_last_error();
        return 1;
    }
    step_end_kernel<<<1, 1, 0, m->st>>>(m->tok, m->tokens, m->pos, m->step, m->seq);
    GD_HIP(hipGetLastError());
    return 0;
}

// Continue a decode after the CPU harness's prefill: take its KV caches and
// position, then generate: out_tokens[0] = first_token and n_gen - 1
// forwards, as nng_generate's loop does. record gets each forward's
// per-layer hidden states ([n_gen - 1][n_layer][n_embd]); seconds the decode
// wall time.
int nngd_decode(nngd_model* m, nng_model* cpu, int32_t first_token, int n_gen, int32_t* out_tokens, float* record,
                double* seconds) {
    const nng_config& c = m->c;
    if (n_gen < 1 || n_gen - 1 > m->n_gen_max) {
        m->err = "n_gen out of range";
        return 1;
    }
    const uint16_t *kc, *vc;
    size_t pos;
    nng_state(cpu, &kc, &vc, &pos, nullptr, nullptr);
    if (pos + (size_t)n_gen > (size_t)c.n_ctx) {
        m->err = "context full";
        return 1;
    }
    const size_t rows = (size_t)c.n_layer * c.n_ctx * c.n_kv, cache = rows * c.head_dim * 2;
    GD_HIP(hipMemcpy(m->kstage, kc, cache, hipMemcpyHostToDevice));
    kperm_kernel<<<(unsigned)((rows * c.head_dim + 255) / 256), 256, 0, m->st>>>(m->kstage, m->kc, rows, c.head_dim);
    GD_HIP(hipGetLastError());
    GD_HIP(hipStreamSynchronize(m->st));
    GD_HIP(hipMemcpy(m->vc, vc, cache, hipMemcpyHostToDevice));
    const uint64_t tok = (uint64_t)first_token;
    const int p = (int)pos, zero = 0;
    GD_HIP(hipMemcpy(m->tok, &tok, 8, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->pos, &p, 4, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->step, &zero, 4, hipMemcpyHostToDevice));
    out_tokens[0] = first_token;
    const int steps = n_gen - 1;
    auto t0 = std::chrono::steady_clock::now();
    if (steps > 0) {
        // Step 0 eagerly; it also settles every lazily sized buffer before capture.
        if (queue_step(m)) return 1;
        GD_HIP(hipStreamSynchronize(m->st));
        if (steps > 1) {
            if (!m->exec) {
                hipGraph_t graph;
                GD_HIP(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal));
                const int rc = queue_step(m);
                hipError_t e = hipStreamEndCapture(m->st, &graph);
                if (rc) return 1;
                GD_HIP(e);
                GD_HIP(hipGraphInstantiate(&m->exec, graph, nullptr, nullptr, 0));
                GD_HIP(hipGraphDestroy(graph));
            }
            for (int s = 1; s < steps; ++s) GD_HIP(hipGraphLaunch(m->exec, m->st));
        }
        GD_HIP(hipStreamSynchronize(m->st));
    }
    auto t1 = std::chrono::steady_clock::now();
    if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
    int ef = 0;
    GD_HIP(hipMemcpy(&ef, m->errf, 4, hipMemcpyDeviceToHost));
    if (ef) {
        m->err = "the device step's hand-off waits ran out";
        return 1;
    }
    if (steps > 0) {
        GD_HIP(hipMemcpy(out_tokens + 1, m->tokens, (size_t)steps * 4, hipMemcpyDeviceToHost));
        if (record)
            GD_HIP(hipMemcpy(record, m->record, (size_t)steps * c.n_layer * c.n_embd * 4, hipMemcpyDeviceToHost));
    }
    return 0;
}

}  // extern "C"
