// The bit-exact f32 path: nncpu's Q8_0 / Q4 gemv with f32 activations, each
// output equal bit for bit to the reference's CPU kernels.
//
// Arithmetic contract (crates/nncpu/src/kernels/scalar.rs:626-742,
// kernels/avx2.rs:1256-1521): a row is 32 independent FMA chains, chain j
// (element j of every 32-block) running over the blocks in order,
//     acc_j = fma(f32(q[32b+j]) * bf16(s[b]), x[32b+j], acc_j),
// where the weight product is exact. The row's result is hsum8 of
// v[l] = (acc_l + acc_{8+l}) + (acc_{16+l} + acc_{24+l}), with
// hsum8(v) = ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)). For Q4 the row adds
// dot_bf16(biases, xsum) (scalar.rs:334-347): an 8-lane FMA accumulator over
// whole groups of 8 blocks, hsum8, then an unfused scalar tail.
//
// GPU mapping: 16 lanes per row, lane j owning chains j and j+16. Four rows
// per wave, sixteen per 256-thread workgroup. The reduction is xor-8 (the
// two accumulator pairs), then xor-4, xor-1, xor-2 (hsum8), which performs
// the reference's additions on the same operands in the same order. No
// split along K: that would change the bits.
//
// Layout (built once at upload, on the device): per row, quants regrouped so
// each lane reads its own bytes with one 128-bit load per group:
//   Q8_0: groups of 8 blocks; lane j's 16 bytes are, for i = 0..7,
//         q[b0+i][j], q[b0+i][j+16].
//   Q4:   groups of 16 blocks; lane j's 16 bytes are byte j of blocks
//         b0..b0+15 (low nibble = chain j, high = chain j+16).
// A row is ngp = ceil(nb / group) whole groups of 256 bytes; the last one is
// zero-filled past block nb (never multiplied: the block loops stop at nb).
// Scales are copied to rows padded to nbp = ngp * group, so a group's scales
// are one aligned 16-byte load per 8.
//
// A second mapping for tall matrices (the lm_head): 8 lanes per row, lane j
// owning chains 4j..4j+3, so one 16-byte load of x serves four chains of a
// block and a wave covers 8 rows. Its quant layout: per row, groups of 128
// bytes (one 16-byte piece per lane),
//   Q8_0: groups of 4 blocks; lane j's piece holds bytes 4j..4j+3 of each.
//   Q4:   groups of 8 blocks; lane j's piece is 4 words, word k holding
//         elements 4j..4j+3 of block 2k in its low nibbles (one per byte)
//         and of block 2k+1 in its high nibbles;
// stored tile-major: for each tile of 32 rows (one workgroup), group g of
// the 32 rows is one 4 KB run, so every wave load reads 1 KB contiguous and
// a workgroup streams one contiguous region. Rows are padded to whole
// groups and tiles with zeros (never multiplied: the block loop stops at
// nb). The reduction becomes xor-2, xor-4 (the accumulator pairs), xor-1
// and an in-lane pair sum (hsum8): the same additions.

#include <algorithm>

#include <type_traits>

#include "common.h"
#include "f32_m1.h"
#include "rmsnorm_exact.h"

namespace nnh {
namespace {

constexpr int Q8_GROUP = 8;
constexpr int Q4_GROUP = 16;

// One thread per destination byte: raw split layout -> per-lane groups.
__global__ void relayout_q8_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ fq, int rows, int nb) {
    const int ngp = (nb + Q8_GROUP - 1) / Q8_GROUP;
    const size_t row_bytes = (size_t)ngp * 256;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * row_bytes) return;
    const size_t r = idx / row_bytes;
    const int d = (int)(idx - r * row_bytes);
    const int g = d >> 8, j = (d >> 4) & 15, k = d & 15;
    const int b = g * Q8_GROUP + (k >> 1), e = j + 16 * (k & 1);
    fq[idx] = b < nb ? raw[r * (size_t)nb * 32 + (size_t)b * 32 + e] : (uint8_t)0;
}

__global__ void relayout_q4_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ fq, int rows, int nb) {
    const int ngp = (nb + Q4_GROUP - 1) / Q4_GROUP;
    const size_t row_bytes = (size_t)ngp * 256;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * row_bytes) return;
    const size_t r = idx / row_bytes;
    const int d = (int)(idx - r * row_bytes);
    const int g = d >> 8, j = (d >> 4) & 15, i = d & 15;
    const int b = g * Q4_GROUP + i;
    fq[idx] = b < nb ? raw[r * (size_t)nb * 16 + (size_t)b * 16 + j] : (uint8_t)0;
}

// The 8-lane layout: one thread per destination word.
__global__ void relayout_q8_v2_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ fq, int rows, int nb) {
    const int ng = (nb + 3) / 4;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // destination word
    const size_t tile_words = (size_t)ng * 32 * 32;
    if (idx >= (size_t)((rows + 31) / 32) * tile_words) return;
    const size_t tile = idx / tile_words;
    const int d = (int)(idx - tile * tile_words);
    const int g = d / 1024, r = (d >> 5) & 31, j = (d >> 2) & 7, i = d & 3;
    const size_t row = tile * 32 + r;
    const int b = 4 * g + i;
    uint32_t v = 0;
    if (b < nb && row < (size_t)rows) v = *(const uint32_t*)(raw + row * (size_t)nb * 32 + (size_t)b * 32 + 4 * j);
    ((uint32_t*)fq)[idx] = v;
}

__global__ void relayout_q4_v2_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ fq, int rows, int nb) {
    const int ng = (nb + 7) / 8;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // destination word
    const size_t tile_words = (size_t)ng * 32 * 32;
    if (idx >= (size_t)((rows + 31) / 32) * tile_words) return;
    const size_t tile = idx / tile_words;
    const int d = (int)(idx - tile * tile_words);
    const int g = d / 1024, r = (d >> 5) & 31, j = (d >> 2) & 7, k = d & 3;
    const size_t rr = tile * 32 + r;
    uint32_t v = 0;
    if (rr >= (size_t)rows) {
        ((uint32_t*)fq)[idx] = 0;
        return;
    }
    const uint8_t* row = raw + rr * (size_t)nb * 16;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int b = 8 * g + 2 * k + half;
        if (b >= nb) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = 4 * j + e;  // element of the block: byte c % 16, high nibble when c >= 16
            const uint32_t nib = (row[(size_t)b * 16 + (c & 15)] >> (c >= 16 ? 4 : 0)) & 15u;
            v |= nib << (8 * e + 4 * half);
        }
    }
    ((uint32_t*)fq)[idx] = v;
}

__global__ void pad_scales_kernel(const uint16_t* __restrict__ s, uint16_t* __restrict__ fs, int rows, int nb,
                                  int nbp) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)rows * nbp;
    if (idx >= total) return;
    size_t r = idx / nbp;
    int b = (int)(idx - r * nbp);
    fs[idx] = b < nb ? s[r * nb + b] : (uint16_t)0;
}

// scalar.rs:355-359: xsum[b] = hsum8 of ((c[l]+c[8+l])+c[16+l])+c[24+l].
__global__ void block_sums_kernel(const float* __restrict__ x, size_t x_stride, int nb, int n_tok,
                                  float* __restrict__ xsum) {
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nb * n_tok) return;
    int t = idx / nb, b = idx - t * nb;
    const float* c = x + (size_t)t * x_stride + 32 * (size_t)b;
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) v[l] = __fadd_rn(__fadd_rn(__fadd_rn(c[l], c[8 + l]), c[16 + l]), c[24 + l]);
    xsum[idx] = __fadd_rn(__fadd_rn(__fadd_rn(v[0], v[4]), __fadd_rn(v[1], v[5])),
                          __fadd_rn(__fadd_rn(v[2], v[6]), __fadd_rn(v[3], v[7])));
}

// Per-token FMA step for the lane's two chains of block b.
template <int M>
__device__ __forceinline__ void step(float (&a0)[M], float (&a1)[M], float w0, float w1, const float* __restrict__ x,
                                     size_t x_stride, size_t e) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float* xm = x + (size_t)m * x_stride + e;
        a0[m] = __builtin_fmaf(w0, xm[0], a0[m]);
        a1[m] = __builtin_fmaf(w1, xm[16], a1[m]);
    }
}

template <int DT, int M>
__global__ __launch_bounds__(256) void gemv_f32_kernel(const uint8_t* __restrict__ fq, const uint16_t* __restrict__ fs,
                                                       const uint16_t* __restrict__ biases,
                                                       const float* __restrict__ x, size_t x_stride,
                                                       const float* __restrict__ xsum, int rows, int nb, int nbp,
                                                       float* __restrict__ y, size_t y_stride) {
    const int j = threadIdx.x & 15;
    const int row_raw = blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool valid = row_raw < rows;
    const int row = valid ? row_raw : rows - 1;  // keep loads in bounds; store is skipped

    float a0[M], a1[M];
#pragma unroll
    for (int m = 0; m < M; ++m) a0[m] = a1[m] = 0.0f;

    const uint16_t* srow = fs + (size_t)row * nbp;
    if (DT == 1) {
        const uint8_t* qrow = fq + (size_t)row * ((nb + Q8_GROUP - 1) / Q8_GROUP) * 256;
        const int ng = nb / Q8_GROUP;
        for (int g = 0; g < ng; ++g) {
            uint4 qv = *(const uint4*)(qrow + (size_t)g * 256 + j * 16);
            uint4 sv = *(const uint4*)(srow + g * Q8_GROUP);
#pragma unroll
            for (int i = 0; i < Q8_GROUP; ++i) {
                float s = bf16f(half_of(sv, i));
                float w0 = (float)(int8_t)byte_of(qv, 2 * i) * s;
                float w1 = (float)(int8_t)byte_of(qv, 2 * i + 1) * s;
                step<M>(a0, a1, w0, w1, x, x_stride, (size_t)32 * (g * Q8_GROUP + i) + j);
            }
        }
        // The partial last group: its first t blocks.
        const int t = nb - ng * Q8_GROUP;
        if (t) {
            uint4 qv = *(const uint4*)(qrow + (size_t)ng * 256 + j * 16);
            uint4 sv = *(const uint4*)(srow + ng * Q8_GROUP);
#pragma unroll
            for (int i = 0; i < Q8_GROUP - 1; ++i) {
                if (i < t) {
                    float s = bf16f(half_of(sv, i));
                    float w0 = (float)(int8_t)byte_of(qv, 2 * i) * s;
                    float w1 = (float)(int8_t)byte_of(qv, 2 * i + 1) * s;
                    step<M>(a0, a1, w0, w1, x, x_stride, (size_t)32 * (ng * Q8_GROUP + i) + j);
                }
            }
        }
    } else {
        const uint8_t* qrow = fq + (size_t)row * ((nb + Q4_GROUP - 1) / Q4_GROUP) * 256;
        const int ng = nb / Q4_GROUP;
        for (int g = 0; g < ng; ++g) {
            uint4 qv = *(const uint4*)(qrow + (size_t)g * 256 + j * 16);
            uint4 s0 = *(const uint4*)(srow + g * Q4_GROUP);
            uint4 s1 = *(const uint4*)(srow + g * Q4_GROUP + 8);
#pragma unroll
            for (int i = 0; i < Q4_GROUP; ++i) {
                float s = bf16f(i < 8 ? half_of(s0, i) : half_of(s1, i - 8));
                uint32_t byte = byte_of(qv, i);
                float w0 = (float)(byte & 15u) * s;
                float w1 = (float)(byte >> 4) * s;
                step<M>(a0, a1, w0, w1, x, x_stride, (size_t)32 * (g * Q4_GROUP + i) + j);
            }
        }
        const int t = nb - ng * Q4_GROUP;
        if (t) {
            uint4 qv = *(const uint4*)(qrow + (size_t)ng * 256 + j * 16);
            uint4 s0 = *(const uint4*)(srow + ng * Q4_GROUP);
            uint4 s1 = *(const uint4*)(srow + ng * Q4_GROUP + 8);
#pragma unroll
            for (int i = 0; i < Q4_GROUP - 1; ++i) {
                if (i < t) {
                    float s = bf16f(i < 8 ? half_of(s0, i) : half_of(s1, i - 8));
                    uint32_t byte = byte_of(qv, i);
                    float w0 = (float)(byte & 15u) * s;
                    float w1 = (float)(byte >> 4) * s;
                    step<M>(a0, a1, w0, w1, x, x_stride, (size_t)32 * (ng * Q4_GROUP + i) + j);
                }
            }
        }
    }

    // Q4 bias term, dot_bf16_f32 (scalar.rs:334-347): lanes 0..7 run the 8
    // accumulator lanes over whole groups of 8 blocks.
    float bdot[M];
    if (DT == 2) {
        const uint16_t* brow = biases + (size_t)row * nb;
        const int body = nb & ~7;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float* xs = xsum + (size_t)m * nb;
            float acc = 0.0f;
            if (j < 8)
                for (int i = j; i < body; i += 8) acc = __builtin_fmaf(bf16f(brow[i]), xs[i], acc);
            // hsum8 over lanes 0..7: xor-4, xor-1, xor-2.
            float p = __fadd_rn(acc, xor_get(acc, 4));
            float q = __fadd_rn(p, xor_get(p, 1));
            float s = __fadd_rn(q, xor_get(q, 2));
            for (int i = body; i < nb; ++i) s = __fadd_rn(s, __fmul_rn(bf16f(brow[i]), xs[i]));
            bdot[m] = s;
        }
    }

#pragma unroll
    for (int m = 0; m < M; ++m) {
        // v[l] = (a0 + a1) + (a2 + a3) at lane l: chains l, 8+l (first
        // accumulators of lanes l and l^8) and 16+l, 24+l (second ones).
        float u = __fadd_rn(a0[m], xor_get(a0[m], 8));
        float w = __fadd_rn(a1[m], xor_get(a1[m], 8));
        float v = __fadd_rn(u, w);
        float p = __fadd_rn(v, xor_get(v, 4));
        float q = __fadd_rn(p, xor_get(p, 1));
        float r = __fadd_rn(q, xor_get(q, 2));
        if (DT == 2) r = __fadd_rn(r, bdot[m]);
        if (valid && j == 0) y[(size_t)m * y_stride + row] = r;
    }
}

typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

// One vector (f32_m1.h). Loads issued before the weights are unconditional
// (clamped indices) and so are the LDS stores that consume them (a clamped
// piece stores its own values again): a conditional store would let the
// compiler sink its load past the weight loads.
constexpr int M1_MAX_NB = 256;                 // x of at most 8192 columns
constexpr int M1_XCH = M1_MAX_NB * 32 / 1024;  // 16-byte x pieces per thread
constexpr int M1W_ROWS = 8;                    // rows per workgroup of the wide kernel
constexpr int M1W_MIN_NB = 64;                 // the wide kernel from 2048 columns

// The Q4 biases of a workgroup's rows and the block sums of x, in LDS.
template <int R>
struct BiasStage {
    static constexpr int K = R * M1_MAX_NB / 256;
    uint16_t v[K];
    int n;
    __device__ __forceinline__ void load(const uint16_t* bi, int row0, int nrows, int nb) {
        n = nrows * nb;
#pragma unroll
        for (int k = 0; k < K; ++k) v[k] = bi[(size_t)row0 * nb + min((int)threadIdx.x + 256 * k, n - 1)];
    }
    __device__ __forceinline__ void store(uint16_t* bl) const {
#pragma unroll
        for (int k = 0; k < K; ++k) bl[min((int)threadIdx.x + 256 * k, n - 1)] = v[k];
    }
};

// 16 lanes per row, 16 rows per workgroup (rows of fewer than M1W_MIN_NB
// blocks: at most 8 Q8 / 4 Q4 groups, all in flight). LDS: x [cols], the
// scale rows [16][nbp]; Q4 adds the block sums [nb] and the biases [16][nb].
template <int DT, int D>
__global__ __launch_bounds__(256) void gemv_f32_m1_kernel(F32Mat m, const float* __restrict__ x,
                                                          float* __restrict__ y) {
    extern __shared__ float lds[];
    const int tid = threadIdx.x, nb = m.nb, cols = nb * 32, n4 = cols / 4;
    const int row0 = blockIdx.x * M1_ROWS, nrows = min(M1_ROWS, m.rows - row0);
    float4 xr[M1W_MIN_NB * 32 / 1024];
#pragma unroll
    for (int k = 0; k < M1W_MIN_NB * 32 / 1024; ++k)
        xr[k] = __builtin_bit_cast(float4, *(const f4u*)(x + 4 * min(tid + 256 * k, n4 - 1)));
    ScaleStage<256, M1_ROWS * M1W_MIN_NB * 2> ss;
    ss.load(m, row0, nrows);
    BiasStage<M1_ROWS> bs;
    if (DT == 2) bs.load(m.bi, row0, nrows, nb);
    const int row_raw = row0 + (tid >> 4);
    const int row = row_raw < m.rows ? row_raw : m.rows - 1;  // keep loads in bounds; the store is skipped
    M1Lane<DT, D> L;
    L.init(m, row, tid & 15);
    // Keep the order: the loads above, then the weights, then the LDS stores
    // that wait for the former only.
    __builtin_amdgcn_sched_barrier(0);
    L.prefetch();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < M1W_MIN_NB * 32 / 1024; ++k) *(float4*)(lds + 4 * min(tid + 256 * k, n4 - 1)) = xr[k];
    uint16_t* sl = (uint16_t*)(lds + cols);
    ss.store(sl);
    float* xs = (float*)(sl + M1_ROWS * m.nbp);
    uint16_t* bl = (uint16_t*)(xs + nb);
    if (DT == 2) bs.store(bl);
    lds_barrier();
    if (DT == 2) {
        for (int b = tid; b < nb; b += 256) xs[b] = m1_block_sum(lds + 32 * b);
        lds_barrier();
    }
    L.run(lds, sl + (row - row0) * m.nbp);
    float r = L.reduce();
    if (DT == 2) r = __fadd_rn(r, m1_bias_dot(bl + (row - row0) * nb, xs, nb, tid & 15));
    if (row_raw < m.rows && (tid & 15) == 0) y[row_raw] = r;
}

// The wide kernel (long rows): 32 lanes per row, 8 rows per workgroup.
// LDS: x transposed [32][S], the scale rows [8][nbp]; Q4 adds the block sums
// [nb] and the biases [8][nb].
template <int DT, int D>
__global__ __launch_bounds__(256) void gemv_f32_m1w_kernel(F32Mat m, const float* __restrict__ x,
                                                           float* __restrict__ y) {
    extern __shared__ float lds[];
    const int tid = threadIdx.x, nb = m.nb, cols = nb * 32, n4 = cols / 4, S = m1w_stride(nb);
    const int row0 = blockIdx.x * M1W_ROWS, nrows = min(M1W_ROWS, m.rows - row0);
    float4 xr[M1_XCH];
#pragma unroll
    for (int k = 0; k < M1_XCH; ++k)
        xr[k] = __builtin_bit_cast(float4, *(const f4u*)(x + 4 * min(tid + 256 * k, n4 - 1)));
    ScaleStage<256, M1W_ROWS * M1_MAX_NB * 2> ss;
    ss.load(m, row0, nrows);
    BiasStage<M1W_ROWS> bs;
    if (DT == 2) bs.load(m.bi, row0, nrows, nb);
    const int row_raw = row0 + (tid >> 5);
    const int row = row_raw < m.rows ? row_raw : m.rows - 1;  // keep loads in bounds; the store is skipped
    M1Wide<DT, D> L;
    L.init(m, row, tid & 31);
    __builtin_amdgcn_sched_barrier(0);
    L.prefetch();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < M1_XCH; ++k) {
        const int p = min(tid + 256 * k, n4 - 1);
        const int b = p >> 3, c = (4 * p) & 31;
        lds[m1w_xpos(b, c, S)] = xr[k].x;
        lds[m1w_xpos(b, c + 1, S)] = xr[k].y;
        lds[m1w_xpos(b, c + 2, S)] = xr[k].z;
        lds[m1w_xpos(b, c + 3, S)] = xr[k].w;
    }
    uint16_t* sl = (uint16_t*)(lds + 32 * S);
    ss.store(sl);
    float* xs = (float*)(sl + M1W_ROWS * m.nbp);
    uint16_t* bl = (uint16_t*)(xs + nb);
    if (DT == 2) bs.store(bl);
    lds_barrier();
    if (DT == 2) {
        for (int b = tid; b < nb; b += 256) {
            float c[32];
#pragma unroll
            for (int e = 0; e < 32; ++e) c[e] = lds[m1w_xpos(b, e, S)];
            xs[b] = m1_block_sum(c);
        }
        lds_barrier();
    }
    L.run(lds, sl + (row - row0) * m.nbp);
    float r = L.reduce();
    if (DT == 2) r = __fadd_rn(r, m1_bias_dot(bl + (row - row0) * nb, xs, nb, tid & 31));
    if (row_raw < m.rows && (tid & 31) == 0) y[row_raw] = r;
}

// The staged kernel (long rows): 1024 threads, at most 8 rows per
// workgroup, about one workgroup per CU. A wave keeps only a few loads in
// flight, so all 16 waves copy x, the rows' scales and the rows' padded
// groups into LDS by direct 1 KB loads (no registers; weight chunk i of row
// r = groups 4i..4i+3, issued in the order c = i * nr + r, copy k of wave w
// being chunk 16 k + w), and the first ceil(nr / 2) waves run the chains
// from LDS, 32 lanes per row as in M1Wide, stage by stage behind the copies:
// once every wave's k-th weight copy has landed, each row holds the groups
// of the first 16 (k + 1) chunks. Every wait is explicit (vmcnt counts a
// wave's copies in issue order); the Q4 biases are the only register loads
// and are consumed after the last wait. The scales are converted to f32 once
// per workgroup, while the weights are still in flight.
constexpr int M1S_NT = 1024;
constexpr int M1S_WAVES = M1S_NT / 64;
constexpr int M1S_ROWS = 8;  // rows per workgroup at most (4 computing waves)

struct M1sLayout {
    int ngp, ng4, nx, ns, SR;  // groups and 1 KB weight chunks per row; x and scale chunks; f32 scale row
    size_t w, x, s, sf, xs, bl, bytes;
    __host__ __device__ M1sLayout(int dt, int nb, int nbp, int nr) {
        const int G = dt == 1 ? 8 : 16;
        ngp = (nb + G - 1) / G;
        ng4 = (ngp + 3) / 4;
        nx = (nb + 7) / 8;
        ns = (nr * nbp * 2 + 1023) / 1024;
        SR = ngp * G;
        w = 0;
        x = w + (size_t)nr * ng4 * 1024;
        s = x + (size_t)nx * 1024;
        sf = s + (size_t)ns * 1024;
        xs = sf + (size_t)nr * SR * 4;
        bl = xs + (size_t)((nb + 3) & ~3) * 4;
        bytes = bl + (dt == 2 ? (size_t)nr * nb * 2 : 0);
    }
};

// s_waitcnt vmcnt(n) for a uniform n in 0..4.
__device__ __forceinline__ void wait_vm_upto4(int n) {
    if (n <= 0)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));
    else if (n == 1)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(1));
    else if (n == 2)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(2));
    else if (n == 3)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(3));
    else
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(4));
}

// One group of a lane's chain: the 16-byte piece, G values of x (row-major
// x, element j: stride 32) and G f32 scales, all from LDS.
template <int DT>
struct M1sGroup {
    static constexpr int G = DT == 1 ? 8 : 16;
    uint4 q;
    float x[G], s[G];
    __device__ __forceinline__ void read(const unsigned char* wrow, const float* xrow, const float* srow, int g) {
        q = *(const uint4*)(wrow + g * 256);
#pragma unroll
        for (int i = 0; i < G; ++i) x[i] = xrow[32 * (g * G + i)];
#pragma unroll
        for (int i = 0; i < G; i += 4) {
            const float4 u = *(const float4*)(srow + g * G + i);
            s[i] = u.x, s[i + 1] = u.y, s[i + 2] = u.z, s[i + 3] = u.w;
        }
    }
    // Blocks i < nblk (all when FULL) into the chain a; h: byte (Q4:
    // nibble) of each pair.
    template <bool FULL>
    __device__ __forceinline__ void run(float& a, int h, int nblk) const {
        const uint32_t dw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < G; ++i) {
            float w;
            if (DT == 1) {
                const uint32_t dd = dw[i >> 1] >> (8 * h);
                w = (float)(int8_t)(dd >> (16 * (i & 1)));
            } else {
                const uint32_t dd = (dw[i >> 2] >> (4 * h)) & 0x0f0f0f0fu;
                w = (float)((dd >> (8 * (i & 3))) & 0xffu);
            }
            if (FULL || i < nblk) a = __builtin_fmaf(w * s[i], x[i], a);
        }
    }
};

// nr_max: the largest row count of a workgroup; K: weight copies per wave,
// ceil(ng4 * nr_max / 16). x must be 16-byte aligned.
template <int DT, int K>
__global__ __launch_bounds__(M1S_NT) void gemv_f32_m1s_kernel(F32Mat m, const float* __restrict__ x,
                                                             float* __restrict__ y, int nr_max) {
    constexpr int G = DT == 1 ? 8 : 16;
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = m.nb;
    const M1sLayout L(DT, nb, m.nbp, nr_max);
    const int row0 = (int)((long)blockIdx.x * m.rows / gridDim.x);
    const int nr = (int)((long)(blockIdx.x + 1) * m.rows / gridDim.x) - row0;

    // Q4 biases (t >> 7, (t & 127) + 128 k) of the rows: registers, stored
    // after the last wait.
    const int br = min(tid >> 7, nr - 1);
    int bb[2];
    uint16_t bv[2];
    if (DT == 2) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            bb[k] = min((tid & 127) + 128 * k, nb - 1);
            bv[k] = m.bi[(size_t)(row0 + br) * nb + bb[k]];
        }
    }

    // x and the scale rows first (32 + 4 chunks at most for nb <= 256).
    const size_t xlen = (size_t)nb * 128, slen = (size_t)nr * m.nbp * 2;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int c = M1S_WAVES * k + wave;
        if (c < L.nx)
            copy_1k(x, xlen, (size_t)c * 1024, smem + L.x + (size_t)c * 1024, lane);
        else if (c < L.nx + L.ns)
            copy_1k(m.fs + (size_t)row0 * m.nbp, slen, (size_t)(c - L.nx) * 1024,
                    smem + L.s + (size_t)(c - L.nx) * 1024, lane);
    }
    // The weights: this wave's kw copies (chunks wave, wave + 16, ...).
    const int nc = L.ng4 * nr;
    const int kw = min(K, (nc - wave + M1S_WAVES - 1) / M1S_WAVES);
    const size_t rbytes = (size_t)L.ngp * 256;
    const uint8_t* wbase = m.fq + (size_t)row0 * rbytes;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int c = M1S_WAVES * k + wave;
        if (c < nc) {
            const int i = c / nr, r = c - i * nr;
            copy_1k(wbase + (size_t)r * rbytes, rbytes, (size_t)i * 1024, smem + L.w + ((size_t)r * L.ng4 + i) * 1024,
                    lane);
        }
    }

    // x and the scales landed (the weights may not have): f32 scales and,
    // for Q4, the block sums of x (waves 4.. never compute).
    wait_vm_upto4(kw);
    lds_barrier();
    float* sf = (float*)(smem + L.sf);
    float* xs = (float*)(smem + L.xs);
    {
        const uint16_t* sb = (const uint16_t*)(smem + L.s);
        for (int e = tid; e < nr * nb; e += M1S_NT) {
            const int r = e / nb, b = e - r * nb;
            sf[r * L.SR + b] = bf16f(sb[r * m.nbp + b]);
        }
        if (DT == 2 && tid >= 256 && tid - 256 < nb)
            xs[tid - 256] = m1_block_sum((const float*)(smem + L.x) + 32 * (tid - 256));
    }

    // The chains: lane j of the row's 32 runs element j; lanes j and j + 16
    // read the same 16-byte piece and take byte (Q4: nibble) h of each pair.
    // Two groups in flight: the next group's LDS reads are issued before the
    // current group's arithmetic.
    const int ncw = (nr + 1) >> 1;
    const int r = min(2 * wave + (lane >> 5), nr - 1), j = lane & 31, h = j >> 4;
    const unsigned char* wrow = smem + L.w + (size_t)r * L.ng4 * 1024 + (j & 15) * 16;
    const float* xrow = (const float*)(smem + L.x) + j;
    const float* srow = sf + r * L.SR;
    const int ng = nb / G;
    float a = 0.0f;
    int glo = 0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        wait_vm_upto4(kw - 1 - k);
        lds_barrier();
        int ghi = L.ngp;
        if (k < K - 1) {
            const int ready = M1S_WAVES * (k + 1) - (nr - 1);
            ghi = ready <= 0 ? 0 : min(L.ngp, 4 * ((ready + nr - 1) / nr));
        }
        if (wave < ncw) {
            const int gf = min(ghi, ng);  // whole groups of this stage: [glo, gf)
            if (glo < gf) {
                M1sGroup<DT> A, B, C;
                A.read(wrow, xrow, srow, glo);
                B.read(wrow, xrow, srow, min(glo + 1, gf - 1));
                __builtin_amdgcn_s_waitcnt(NNH_LGKMCNT0);
                int g = glo;
                for (; g + 2 < gf; g += 3) {
                    C.read(wrow, xrow, srow, g + 2);
                    __builtin_amdgcn_sched_barrier(0);
                    A.template run<true>(a, h, G);
                    __builtin_amdgcn_sched_barrier(0);
                    A.read(wrow, xrow, srow, min(g + 3, gf - 1));
                    __builtin_amdgcn_sched_barrier(0);
                    B.template run<true>(a, h, G);
                    __builtin_amdgcn_sched_barrier(0);
                    B.read(wrow, xrow, srow, min(g + 4, gf - 1));
                    __builtin_amdgcn_sched_barrier(0);
                    C.template run<true>(a, h, G);
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (g < gf) A.template run<true>(a, h, G);
                if (g + 1 < gf) B.template run<true>(a, h, G);
            }
            if (ghi == L.ngp && ng < L.ngp && glo <= ng) {
                M1sGroup<DT> A;
                A.read(wrow, xrow, srow, ng);
                A.template run<false>(a, h, nb - ng * G);
            }
        }
        glo = ghi;
    }
    uint16_t* bl = (uint16_t*)(smem + L.bl);
    if (DT == 2) {
#pragma unroll
        for (int k = 0; k < 2; ++k) bl[br * nb + bb[k]] = bv[k];
        lds_barrier();
    }
    if (wave >= ncw) return;
    const float u = __fadd_rn(a, xor_get(a, 8));
    const float v = __fadd_rn(u, xor_get(u, 16));
    const float p = __fadd_rn(v, xor_get(v, 4));
    const float q = __fadd_rn(p, xor_get(p, 1));
    float res = __fadd_rn(q, xor_get(q, 2));
    if (DT == 2) res = __fadd_rn(res, m1_bias_dot(bl + r * nb, xs, nb, j));
    if (2 * wave + (lane >> 5) < nr && j == 0) y[row0 + 2 * wave + (lane >> 5)] = res;
}

// The streamed kernel (long rows, many of them): 32 lanes per row, lane j
// running chain j alone (M1Wide's arithmetic on the same 16-lane layout),
// every wave computing two rows; a workgroup takes NT / 32 consecutive rows.
// x is staged once per workgroup. Each lane streams its row's groups
// straight from global memory into a ring of PF register slots (the quant
// piece and the group's BF16 scales, the scale loads the same address
// across the row's 32 lanes), so PF groups are always in flight behind the
// arithmetic; the staged kernel's LDS copies of every row are not needed.
// The lane's byte (Q8) or nibble (Q4) of each pair is brought to fixed
// positions once per group.
constexpr int M1R_MIN_ROWS = 2048;  // fills the GPU at 32 lanes per row

// One group in flight: the quant piece, the group's BF16 scales and, for
// Q4, the two biases that the lane's bias-dot lane (j mod 8) takes from the
// group (blocks 16g + j mod 8 and 16g + 8 + j mod 8).
template <int DT>
struct M1xSlot {
    static constexpr int G = DT == 1 ? 8 : 16;
    uint4 q;
    uint4 s[G / 8];
    float4 sf[G / 4];  // the scales as f32 (staged rows)
    uint32_t b0, b1;   // Q4 only
};

// Group g's quant piece and scales; Q4: the biases of group gb (g clamped
// to the row's whole groups, so that those loads stay inside the row).
template <int DT, bool SL>
__device__ __forceinline__ void m1x_load(M1xSlot<DT>& sl, const uint8_t* qrow, const uint16_t* srow,
                                         const uint16_t* brow, int g, int gb) {
    constexpr int G = DT == 1 ? 8 : 16;
    sl.q = load_nt16u(qrow + (size_t)g * 256);
    if (!SL)
#pragma unroll
        for (int k = 0; k < G / 8; ++k) sl.s[k] = *(const uint4*)(srow + g * G + 8 * k);
    if (DT == 2) {
        sl.b0 = brow[16 * gb];
        sl.b1 = brow[16 * gb + 8];
    }
}

// One group of the lane's chain with x in its natural order in LDS (xb: x
// at the group's first block plus the lane's element; block i's value 32
// floats on). Q4 whole groups also take the group's two steps of the lane's
// bias-dot accumulator (xsg: the block sums at the group's first block plus
// j mod 8).
// SF: the group's scales are in sl.sf as f32, else in sl.s as BF16.
template <int DT, bool FULL, bool SF = false>
__device__ __forceinline__ void m1x_group(const M1xSlot<DT>& sl, const float* xb, const float* xsg, int h, int nblk,
                                          float& a, float& ab) {
    constexpr int G = DT == 1 ? 8 : 16;
    uint32_t qd[4] = {sl.q.x, sl.q.y, sl.q.z, sl.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        qd[k] = DT == 1 ? qd[k] >> (8 * h) : (qd[k] >> (4 * h)) & 0x0f0f0f0fu;
        if (DT == 2) asm volatile("" : "+v"(qd[k]));
    }
    float xv[G];
#pragma unroll
    for (int i = 0; i < G; ++i)
        if (FULL || i < nblk) xv[i] = xb[32 * i];
    if (DT == 2 && FULL) {
        ab = __builtin_fmaf(bf16f(sl.b0), xsg[0], ab);
        ab = __builtin_fmaf(bf16f(sl.b1), xsg[8], ab);
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
        if (FULL || i < nblk) {
            const float4 f4 = sl.sf[i / 4];
            const float sb = SF ? (i % 4 == 0 ? f4.x : i % 4 == 1 ? f4.y : i % 4 == 2 ? f4.z : f4.w)
                                : bf16f(half_of(sl.s[i / 8], i % 8));
            float w;
            if (DT == 1)
                w = (float)(int8_t)((qd[i >> 1] >> (16 * (i & 1))) & 0xffu);
            else
                w = (float)((qd[i >> 2] >> (8 * (i & 3))) & 0xffu);
            a = __builtin_fmaf(w * sb, xv[i], a);
        }
    }
}

// LDS of the streamed kernel: x (nb * 128 bytes, rounded up to
// whole 1 KB copies), the scale rows of the workgroup's rpw rows as copied
// (BF16) and, Q4, as f32 (each rounded up likewise), then the Q4 block sums
// of x (nb floats).
__host__ __device__ inline size_t m1x_x_bytes(int nb) { return ((size_t)nb * 128 + 1023) & ~(size_t)1023; }
__host__ __device__ inline size_t m1x_s_bytes(int nbp, int rpw) {
    return ((size_t)rpw * nbp * 2 + 1023) & ~(size_t)1023;
}
__host__ __device__ inline size_t m1x_sf_bytes(int nbp, int rpw) {
    return ((size_t)rpw * nbp * 4 + 1023) & ~(size_t)1023;
}
inline size_t m1x_lds(int dt, int nb, int nbp, int rpw, bool norm = false) {
    // NORM: x, then r (1 KB wider: it then holds the sum of squares'
    // chain-major copy), then gamma.
    return m1x_x_bytes(nb) * (norm ? 3 : 1) + (norm ? 1024 : 0) + m1x_s_bytes(nbp, rpw) +
           (dt == 2 ? m1x_sf_bytes(nbp, rpw) + (size_t)nb * 4 : 0);
}

// The fused residual add and RMSNorm (NormIn) on a vector of `cols` floats
// staged in LDS at v, with r and gamma staged at rw and gw (r's copy unused
// when n.r is NULL); nt threads. Afterwards v holds the gemv's input. The
// operations and their order are the device forward's resid_norm_kernel's
// (forward.rs:719-841: the add, sum_sq, the scale, (v * scale) * gamma).
template <int B>
__device__ __forceinline__ void norm_prologue(const NormIn& n, float* v, float* rw, const float* gw, int cols,
                                              float* sc_lds, int nt) {
    const int tid = threadIdx.x;
    for (int i = 4 * tid; i < cols; i += 4 * nt) {
        float4 a = *(const float4*)(v + i);
        if (n.r) {
            const float4 b = *(const float4*)(rw + i);
            a = float4{__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w)};
            *(float4*)(v + i) = a;
        }
        if (blockIdx.x == 0) {
            if (n.x_out) *(float4*)(n.x_out + i) = a;
            if (n.rec) *(float4*)(n.rec + i) = a;
        }
    }
    __syncthreads();
    // v chain-major over r's region (r is read by now): element e at
    // (e mod 8) * ts + e / 8, so the chain's lanes read 16 bytes at a time.
    const int ts = rms_t_stride(cols);
    for (int i = 4 * tid; i < cols; i += 4 * nt) {
        const float4 a = *(const float4*)(v + i);
        const int p = i >> 2;
        float* d = rw + (size_t)(4 * (p & 1)) * ts + (p >> 1);
        d[0] = a.x;
        d[ts] = a.y;
        d[2 * ts] = a.z;
        d[3 * ts] = a.w;
    }
    __syncthreads();
    if (tid < 64) {
        const double ss = rms_sumsq_t<B>(rw, cols, tid);
        if (tid == 0) *sc_lds = rms_scale(ss, cols, n.eps);
    }
    __syncthreads();
    const float sc = *sc_lds;
    for (int i = 4 * tid; i < cols; i += 4 * nt) {
        const float4 a = *(const float4*)(v + i), g = *(const float4*)(gw + i);
        *(float4*)(v + i) = float4{__fmul_rn(__fmul_rn(a.x, sc), g.x), __fmul_rn(__fmul_rn(a.y, sc), g.y),
                                   __fmul_rn(__fmul_rn(a.z, sc), g.z), __fmul_rn(__fmul_rn(a.w, sc), g.w)};
    }
    __syncthreads();
}

// x is copied to LDS as it lies in memory: every wave issues its share of
// 1 KB direct-to-LDS copies of x (and, SL, of the workgroup's scale rows:
// one contiguous span) before the first PF groups of its row, so the
// staging is one round trip and holds no registers. A lane reads block b's
// element j at 32 b + j (the 32 lanes of a row read 128 contiguous bytes).
// Q4: the block sums of x are formed from the LDS copy after the staging
// barrier, and the bias dot (dot_bf16_f32, scalar.rs:334-347: lane j mod 8
// of the accumulator over whole groups of 8 blocks, hsum8, the unfused
// tail) runs alongside the chains, its biases streamed with the weights.
template <int DT, int NT, int M1R_PF, bool SL, bool NORM>
__global__ __launch_bounds__(NT) void gemv_f32_m1x_kernel(F32Mat m, const float* __restrict__ x,
                                                         float* __restrict__ y, NormIn nrm) {
    constexpr int G = DT == 1 ? 8 : 16;
    const int nt = blockDim.x;  // at most NT: 32 lanes per row
    const int RPW = nt >> 5;    // rows per workgroup
    const int NW = nt >> 6;
    extern __shared__ __align__(1024) unsigned char m1x_smem[];
    __shared__ float nsc;  // the norm's scale (NORM)
    const int tid = threadIdx.x, nb = m.nb, wave = tid >> 6, lane = tid & 63;
    const int ngp = m1_groups(DT, nb), ng = nb / G;
    const size_t XB = m1x_x_bytes(nb), XR = NORM ? 3 * XB + 1024 : XB;  // x (NORM: then r, 1 KB wider, and gamma)
    float* xw = (float*)m1x_smem;
    // Q4 with the scale rows staged (SF): the chains read them as f32,
    // converted once per workgroup (Q4 1-4 % faster at the measured
    // shape; Q8, whose groups hold half the blocks, 5-12 % slower: twice the
    // LDS reads of its scales), else each lane converts its BF16 scales.
    constexpr bool SF = SL && DT == 2;
    const uint16_t* scl = (const uint16_t*)(m1x_smem + XR);
    float* sclf = (float*)(m1x_smem + XR + (SL ? m1x_s_bytes(m.nbp, RPW) : 0));  // the scale rows as f32 (SF)
    float* xs = (float*)(m1x_smem + XR + (SL ? m1x_s_bytes(m.nbp, RPW) + (SF ? m1x_sf_bytes(m.nbp, RPW) : 0) : 0));
    const int row0 = blockIdx.x * RPW;
    const int rraw = row0 + (tid >> 5);
    const int row = rraw < m.rows ? rraw : m.rows - 1;
    const int j = tid & 31, h = j >> 4, j8 = j & 7;

    {
        const size_t xl = (size_t)nb * 128;
        const float* src = NORM ? nrm.x : x;
        for (size_t c = wave; c * 1024 < xl; c += NW) copy_1k(src, xl, c * 1024, m1x_smem + c * 1024, lane);
        if (NORM) {
            if (nrm.r)
                for (size_t c = wave; c * 1024 < xl; c += NW) copy_1k(nrm.r, xl, c * 1024, m1x_smem + XB + c * 1024, lane);
            for (size_t c = wave; c * 1024 < xl; c += NW)
                copy_1k(nrm.gamma, xl, c * 1024, m1x_smem + 2 * XB + 1024 + c * 1024, lane);
        }
        if (SL) {
            // The scale rows of the workgroup's rows: one contiguous span.
            const size_t sl_len = (size_t)min(RPW, m.rows - row0) * m.nbp * 2;
            const unsigned char* ssrc = (const unsigned char*)(m.fs + (size_t)row0 * m.nbp);
            for (size_t c = wave; c * 1024 < sl_len; c += NW)
                copy_1k(ssrc, sl_len, c * 1024, m1x_smem + XR + c * 1024, lane);
        }
    }
    const uint4* srl = (const uint4*)(scl + (size_t)(row - row0) * m.nbp);       // the row's scales in LDS
    const float4* srf = (const float4*)(sclf + (size_t)(row - row0) * m.nbp);  // as f32 (SF)
    const uint8_t* qrow = m.fq + (size_t)row * ngp * 256 + (j & 15) * 16;
    const uint16_t* srow = m.fs + (size_t)row * m.nbp;
    // Q4: block 16g + j8 of the row's biases; whole groups only, so the
    // clamped prefetches past them read inside the row's first ng groups.
    const uint16_t* brow = DT == 2 ? m.bi + (size_t)row * nb + j8 : nullptr;
    const int ngb = ng > 0 ? ng : 1;  // bias prefetches stay in whole groups (or group 0)
    M1xSlot<DT> slot[M1R_PF];
#pragma unroll
    for (int d = 0; d < M1R_PF; ++d) {
        const int g = d < ngp ? d : ngp - 1;
        m1x_load<DT, SL>(slot[d], qrow, srow, brow, g, min(g, ngb - 1));
    }
    // The copies have landed once at most the slots' loads are in flight
    // (per slot: the quant piece, the scales unless staged, Q4's two
    // biases); the norm and the block sums run while the slots fill.
    wait_vm_keep<M1R_PF * (1 + (SL ? 0 : G / 8) + (DT == 2 ? 2 : 0))>(m.fq, m.fs, m.bi);
    __syncthreads();
    if (SF) {
        // The staged scale rows to f32 once per workgroup, so the chains
        // take each scale as it is instead of converting it per lane.
        const int pairs = min(RPW, m.rows - row0) * m.nbp / 2;
        for (int e = tid; e < pairs; e += nt) {
            const uint32_t w = ((const uint32_t*)scl)[e];
            ((float2*)sclf)[e] = float2{bf16f(w & 0xffffu), bf16f(w >> 16)};
        }
    }
    if (NORM)
        norm_prologue<8>(nrm, xw, (float*)(m1x_smem + XB), (const float*)(m1x_smem + 2 * XB + 1024), nb * 32,
                          &nsc, nt);
    if (DT == 2)
        for (int b = tid; b < nb; b += nt) xs[b] = m1_block_sum(xw + 32 * b);
    if (DT == 2) lds_barrier();

    const float* xp = xw + j;
    float a = 0.0f, ab = 0.0f;
    int g = 0;
    for (; g + M1R_PF <= ng; g += M1R_PF) {
#pragma unroll
        for (int d = 0; d < M1R_PF; ++d) {
            if (SF)
#pragma unroll
                for (int k = 0; k < G / 4; ++k) slot[d].sf[k] = srf[(g + d) * (G / 4) + k];
            else if (SL)
#pragma unroll
                for (int k = 0; k < G / 8; ++k) slot[d].s[k] = srl[(g + d) * (G / 8) + k];
            m1x_group<DT, true, SF>(slot[d], xp + (g + d) * G * 32, xs + (g + d) * G + j8, h, G, a, ab);
            const int gn = min(g + d + M1R_PF, ngp - 1);
            m1x_load<DT, SL>(slot[d], qrow, srow, brow, gn, min(gn, ngb - 1));
        }
    }
#pragma unroll
    for (int d = 0; d < M1R_PF; ++d) {
        if (SF && g + d < ngp)
#pragma unroll
            for (int k = 0; k < G / 4; ++k) slot[d].sf[k] = srf[(g + d) * (G / 4) + k];
        else if (SL && g + d < ngp)
#pragma unroll
            for (int k = 0; k < G / 8; ++k) slot[d].s[k] = srl[(g + d) * (G / 8) + k];
        if (g + d < ng)
            m1x_group<DT, true, SF>(slot[d], xp + (g + d) * G * 32, xs + (g + d) * G + j8, h, G, a, ab);
        else if (g + d == ng && ng < ngp)
            m1x_group<DT, false, SF>(slot[d], xp + (g + d) * G * 32, xs, h, nb - ng * G, a, ab);
    }
    const float u = __fadd_rn(a, xor_get(a, 8));
    const float v = __fadd_rn(u, xor_get(u, 16));
    const float p = __fadd_rn(v, xor_get(v, 4));
    const float q = __fadd_rn(p, xor_get(p, 1));
    float res = __fadd_rn(q, xor_get(q, 2));
    if (DT == 2) {
        // The bias dot's blocks past the whole groups: the rest of the
        // 8-block body, hsum8, then the unfused tail.
        const uint16_t* bfull = m.bi + (size_t)row * nb;
        const int body = nb & ~7;
        for (int i = G * ng + j8; i < body; i += 8) ab = __builtin_fmaf(bf16f(bfull[i]), xs[i], ab);
        const float bp = __fadd_rn(ab, xor_get(ab, 4));
        const float bq = __fadd_rn(bp, xor_get(bp, 1));
        float bs = __fadd_rn(bq, xor_get(bq, 2));
        for (int i = body; i < nb; ++i) bs = __fadd_rn(bs, __fmul_rn(bf16f(bfull[i]), xs[i]));
        res = __fadd_rn(res, bs);
    }
    if (rraw < m.rows && j == 0) y[rraw] = res;
}

// The streamed kernel's conditions: enough rows to fill the GPU at 32 lanes
// per row, x (staged whole in LDS) at most 64 KB and 16-byte aligned.
// x staged whole: up to 150 KB of LDS (rows of about 37000 columns).
constexpr size_t M1R_MAX_LDS = 150 * 1024;
constexpr size_t CU_LDS_BYTES = 160 * 1024;  // LDS of one gfx950 CU
static bool m1r_fits(int dt, int rows, int nb, const float* x) {
    const int nbp = dt == 1 ? (nb + 7) / 8 * 8 : (nb + 15) / 16 * 16;
    return nb >= M1W_MIN_NB && rows >= M1R_MIN_ROWS && m1x_lds(dt, nb, nbp, 8) <= M1R_MAX_LDS &&
           ((uintptr_t)x & 15) == 0;
}
// The streamed kernel's instances may take more than the default 64 KB of
// dynamic LDS (set once per instance).
template <int DT, int NT, int PF, bool SL, bool NORM>
static void m1x_allow_lds() {
    static const bool once = [] {
        return hipFuncSetAttribute((const void*)gemv_f32_m1x_kernel<DT, NT, PF, SL, NORM>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)M1R_MAX_LDS) == hipSuccess;
    }();
    (void)once;
}

// The streamed kernel's rows per workgroup: every CU takes the same rows
// where the matrix has at most 32 per CU (ceil(rows / CUs), even, at least
// 8: 3584 rows as 256 workgroups of 14, 4608 as 256 of 18, where fixed
// 8- or 16-row workgroups left some CUs a second one), else 16. Prefetch
// depth: 3 groups (48 blocks) for Q4, 6 (48 blocks) for Q8 (deeper
// measured slower at Llama's and Qwen's shapes). The rows' scales are
// staged in LDS too unless that would leave fewer workgroups resident per
// CU than the launch needs (long rows: the copy of x alone takes half of a
// CU's LDS). NORM: the fused residual add and RMSNorm first (x unused; its
// input is nrm's).
template <int DT, int NT, bool NORM>
void launch_m1x_nt(const F32Mat& m, const float* x, float* y, const NormIn& nrm, bool sl, int rpw, size_t lds,
                   hipStream_t st) {
    constexpr int PF = DT == 1 ? 6 : 3;
    const dim3 grid(ceil_div(m.rows, rpw)), block(rpw * 32);
    if (sl) {
        m1x_allow_lds<DT, NT, PF, true, NORM>();
        gemv_f32_m1x_kernel<DT, NT, PF, true, NORM><<<grid, block, lds, st>>>(m, x, y, nrm);
    } else if constexpr (NT <= 512) {  // (1024 threads leave too few registers for the scales' loads)
        m1x_allow_lds<DT, NT, PF, false, NORM>();
        gemv_f32_m1x_kernel<DT, NT, PF, false, NORM><<<grid, block, lds, st>>>(m, x, y, nrm);
    }
}

template <int DT, bool NORM>
void launch_m1x(const F32Mat& m, const float* x, float* y, const NormIn& nrm, hipStream_t st) {
    const int rows = m.rows, nb = m.nb, nbp = m.nbp, cus = cu_count();
    int rpw = 16;
    if (rows <= 32 * cus) {
        rpw = ceil_div(rows, cus);
        rpw += rpw & 1;
        if (rpw < 8) rpw = 8;
    }
    const auto staged = [&](int r) {
        const int need = ceil_div(ceil_div(rows, r), cus);
        const size_t lds_sl = m1x_lds(DT, nb, nbp, r, NORM);
        const int fit = (int)(CU_LDS_BYTES / m1x_lds(DT, nb, nbp, 0, NORM));
        return lds_sl <= M1R_MAX_LDS && (int)(CU_LDS_BYTES / lds_sl) >= std::min(need, fit);
    };
    bool sl = staged(rpw);
    if (!sl && rpw > 16) {  // more than 16 rows only with the scales staged
        rpw = 16;
        sl = staged(rpw);
    }
    const size_t lds = m1x_lds(DT, nb, nbp, sl ? rpw : 0, NORM);
    if (rpw <= 8)
        launch_m1x_nt<DT, 256, NORM>(m, x, y, nrm, sl, rpw, lds, st);
    else if (rpw <= 16)
        launch_m1x_nt<DT, 512, NORM>(m, x, y, nrm, sl, rpw, lds, st);
    else
        launch_m1x_nt<DT, 1024, NORM>(m, x, y, nrm, sl, rpw, lds, st);
}

// Weight-load slots D >= the row's groups: 4 or 8 (Q4: 2 or 4) for the
// 16-lane kernel, 8, 16 or 32 (Q4: up to 16) for the wide one.
template <int DT>
void launch_m1(const uint8_t* fq, const uint16_t* fs, const uint16_t* bi, const float* x, int rows, int nb, int nbp,
               float* y, hipStream_t st) {
    const F32Mat m{fq, fs, bi, rows, nb, nbp};
    const int ngp = DT == 1 ? (nb + 7) / 8 : (nb + 15) / 16;
    const size_t q4 = DT == 2 ? (size_t)nb * 4 : 0;
    const dim3 block(256);
    if (m1r_fits(DT, rows, nb, x)) {
        launch_m1x<DT, false>(m, x, y, NormIn{}, st);
        return;
    }
    if (nb >= M1W_MIN_NB) {
        // About one workgroup per CU, at most M1S_ROWS rows each.
        const int nwg = std::max(std::min(rows, cu_count()), ceil_div(rows, M1S_ROWS));
        const int nr = ceil_div(rows, nwg);
        const M1sLayout L(DT, nb, nbp, nr);
        const int k = ceil_div((long)L.ng4 * nr, M1S_WAVES);
        const dim3 g(nwg), b(M1S_NT);
        if (((uintptr_t)x & 15) == 0 && k <= 4) {
            if (k <= 1)
                gemv_f32_m1s_kernel<DT, 1><<<g, b, L.bytes, st>>>(m, x, y, nr);
            else if (k == 2)
                gemv_f32_m1s_kernel<DT, 2><<<g, b, L.bytes, st>>>(m, x, y, nr);
            else if (k == 3)
                gemv_f32_m1s_kernel<DT, 3><<<g, b, L.bytes, st>>>(m, x, y, nr);
            else
                gemv_f32_m1s_kernel<DT, 4><<<g, b, L.bytes, st>>>(m, x, y, nr);
            return;
        }
    }
    if (nb >= M1W_MIN_NB) {
        const size_t S = ((nb + 3) & ~3) + (((nb + 3) & 4) ? 0 : 4);
        const size_t lds = 32 * S * 4 + (size_t)M1W_ROWS * nbp * 2 + q4 + (DT == 2 ? (size_t)M1W_ROWS * nb * 2 : 0);
        const dim3 grid(ceil_div(rows, M1W_ROWS));
        if (ngp <= 8)
            gemv_f32_m1w_kernel<DT, 8><<<grid, block, lds, st>>>(m, x, y);
        else if (ngp <= 16)
            gemv_f32_m1w_kernel<DT, 16><<<grid, block, lds, st>>>(m, x, y);
        else
            gemv_f32_m1w_kernel<DT, 32><<<grid, block, lds, st>>>(m, x, y);
        return;
    }
    const size_t lds = (size_t)nb * 32 * 4 + (size_t)M1_ROWS * nbp * 2 + q4 + (DT == 2 ? (size_t)M1_ROWS * nb * 2 : 0);
    const dim3 grid(ceil_div(rows, M1_ROWS));
    if (ngp <= (DT == 1 ? 4 : 2))
        gemv_f32_m1_kernel<DT, DT == 1 ? 4 : 2><<<grid, block, lds, st>>>(m, x, y);
    else
        gemv_f32_m1_kernel<DT, DT == 1 ? 8 : 4><<<grid, block, lds, st>>>(m, x, y);
}

// The 8-lane mapping (tall matrices).

constexpr int V2_R = 4;  // rows per lane group of the multi-vector form on tall matrices

// One block for the lane group's R rows: w[r][e] (exact weights) against
// x[32b + 4j + e] of every token, read from the workgroup's LDS copy of x
// (LDS reads wait on their own counter, so they never wait for the weight
// loads in flight).
template <int R, int M>
__device__ __forceinline__ void v2_block(float (&acc)[R][M][4], const float (&w)[R][4], const float* xl, int cols,
                                         int e0) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float4 xv = *(const float4*)(xl + m * cols + e0);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r][m][0] = __builtin_fmaf(w[r][0], xv.x, acc[r][m][0]);
            acc[r][m][1] = __builtin_fmaf(w[r][1], xv.y, acc[r][m][1]);
            acc[r][m][2] = __builtin_fmaf(w[r][2], xv.z, acc[r][m][2]);
            acc[r][m][3] = __builtin_fmaf(w[r][3], xv.w, acc[r][m][3]);
        }
    }
}

// One group of the lane's rows in flight: the 16-byte quant pieces and the
// group's BF16 scales (Q8: 4, in s.x and s.y; Q4: 8).
template <int DT, int R>
struct V2Group {
    uint4 q[R];
    typename std::conditional<DT == 1, uint2, uint4>::type s[R];
};

template <int DT, int R>
__device__ __forceinline__ void v2_load(V2Group<DT, R>& gr, const uint4* const (&qrow)[R],
                                        const uint16_t* const (&srow)[R], int g) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        gr.q[r] = load_nt16u(qrow[r] + (size_t)g * 32 * 8);
        if constexpr (DT == 1)
            gr.s[r] = *(const uint2*)(srow[r] + 4 * g);
        else
            gr.s[r] = *(const uint4*)(srow[r] + 8 * g);
    }
}

__device__ __forceinline__ uint32_t half2_of(const uint2& v, int i) {
    return ((i < 2 ? v.x : v.y) >> (16 * (i & 1))) & 0xffffu;
}

// The exact weights of block i of the group for the lane's R rows
// (elements 4j..4j+3).
template <int DT, int R>
__device__ __forceinline__ void v2_weights(float (&w)[R][4], const V2Group<DT, R>& gr, int i) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if constexpr (DT == 1) {
            const uint32_t qw = i == 0 ? gr.q[r].x : i == 1 ? gr.q[r].y : i == 2 ? gr.q[r].z : gr.q[r].w;
            const float s = bf16f(half2_of(gr.s[r], i));
#pragma unroll
            for (int e = 0; e < 4; ++e) w[r][e] = (float)(int8_t)(qw >> (8 * e)) * s;  // exact
        } else {
            const int k = i >> 1, half = i & 1;
            const uint32_t qw = k == 0 ? gr.q[r].x : k == 1 ? gr.q[r].y : k == 2 ? gr.q[r].z : gr.q[r].w;
            uint32_t nib = (qw >> (4 * half)) & 0x0f0f0f0fu;
            // Opaque to the compiler: it would fold the mask into a bit-field
            // extract per element instead of converting the bytes directly.
            asm volatile("" : "+v"(nib));
            const float s = bf16f(half_of(gr.s[r], i));
#pragma unroll
            for (int e = 0; e < 4; ++e) w[r][e] = (float)((nib >> (8 * e)) & 0xffu) * s;  // exact
        }
    }
}

// Blocks G*g .. G*g + G - 1 (those below nb unless FULL). One vector: the
// group's x pieces are read from LDS first, so one wait covers the group.
template <int DT, int R, int M, bool FULL>
__device__ __forceinline__ void v2_group(float (&acc)[R][M][4], const V2Group<DT, R>& gr, int g, int nb,
                                         const float* xl, int j) {
    constexpr int G = DT == 1 ? 4 : 8;
    if constexpr (M == 1) {
        float4 xv[G];
#pragma unroll
        for (int i = 0; i < G; ++i)
            if (FULL || G * g + i < nb) xv[i] = *(const float4*)(xl + 32 * (G * g + i) + 4 * j);
#pragma unroll
        for (int i = 0; i < G; ++i) {
            if (!FULL && G * g + i >= nb) break;
            float w[R][4];
            v2_weights<DT, R>(w, gr, i);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                acc[r][0][0] = __builtin_fmaf(w[r][0], xv[i].x, acc[r][0][0]);
                acc[r][0][1] = __builtin_fmaf(w[r][1], xv[i].y, acc[r][0][1]);
                acc[r][0][2] = __builtin_fmaf(w[r][2], xv[i].z, acc[r][0][2]);
                acc[r][0][3] = __builtin_fmaf(w[r][3], xv[i].w, acc[r][0][3]);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const int b = G * g + i;
            if (!FULL && b >= nb) break;
            float w[R][4];
            v2_weights<DT, R>(w, gr, i);
            v2_block<R, M>(acc, w, xl, nb * 32, 32 * b + 4 * j);
        }
    }
}

// Workgroup: 4 waves = 32 lane groups; lane group lg of workgroup wg runs
// rows (wg * R + r) * 32 + lg for r < R, one row from each of R consecutive
// 32-row tiles (R rows share every x read; fewer rows per lane group give
// more waves to a shorter matrix). PF groups of weights are in flight per
// lane: group g in slot g % PF, each slot refilled with the group PF ahead
// right after its arithmetic.
template <int DT, int M, int R, int PF, bool NORM = false>
__global__ __launch_bounds__(256) void gemv_f32_v2_kernel(const uint8_t* __restrict__ fq,
                                                          const uint16_t* __restrict__ fs,
                                                          const uint16_t* __restrict__ biases,
                                                          const float* __restrict__ x, size_t x_stride,
                                                          const float* __restrict__ xsum, int rows, int nb, int nbp,
                                                          float* __restrict__ y, size_t y_stride,
                                                          uint64_t* __restrict__ part, NormIn nrm) {
    static_assert(!NORM || M == 1, "the fused norm takes one vector");
    constexpr int G = DT == 1 ? 4 : 8;
    const int j = threadIdx.x & 7, lg = threadIdx.x >> 3;
    const int ng = (nb + G - 1) / G;
    int row[R];
    const uint4* qrow[R];
    const uint16_t* srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int tile = blockIdx.x * R + r;
        const int raw = tile * 32 + lg;
        row[r] = raw < rows ? raw : rows - 1;  // keep loads in bounds; stores are skipped
        const int t = row[r] / 32;
        // Tile-major: group g of this row at ((tile * ng + g) * 32 + row % 32) * 128.
        qrow[r] = (const uint4*)(fq + ((size_t)t * ng * 32 + (row[r] % 32)) * 128) + j;
        srow[r] = fs + (size_t)row[r] * nbp;
    }

    float acc[R][M][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[r][m][e] = 0.0f;

    V2Group<DT, R> slot[PF];
    constexpr int PF0 = PF == 2 ? 1 : PF;  // groups issued before the arithmetic
    // [M][cols] (NORM: x, then r or gamma one 1 KB-rounded region on),
    // 16-byte aligned for float4.
    extern __shared__ __align__(16) float xl[];
    const int cols = nb * 32;
    if constexpr (NORM) {
        // x and r (else gamma) are copied to LDS, then the first weight
        // groups issued: the add and the sum of squares run while those are
        // in flight. With r, gamma is copied over r's region once the add
        // is done, alongside the sum of squares.
        __shared__ float nsc;
        const size_t xlen = (size_t)cols * 4, xb = m1x_x_bytes(nb);
        unsigned char* l8 = (unsigned char*)xl;
        float* gl = (float*)(l8 + xb);
        const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
        for (size_t c = wave; c * 1024 < xlen; c += 4) copy_1k(nrm.x, xlen, c * 1024, l8 + c * 1024, lane);
        const float* second = nrm.r ? nrm.r : nrm.gamma;
        for (size_t c = wave; c * 1024 < xlen; c += 4) copy_1k(second, xlen, c * 1024, l8 + xb + c * 1024, lane);
#pragma unroll
        for (int d = 0; d < PF0; ++d) v2_load<DT, R>(slot[d], qrow, srow, d < ng ? d : ng - 1);
        wait_vm_keep<PF0 * 2 * R>(fq, fs);  // per group and row: the quant piece and the scales
        __syncthreads();
        for (int i = 4 * tid; i < cols; i += 4 * 256) {
            float4 a = *(const float4*)(xl + i);
            if (nrm.r) {
                const float4 b = *(const float4*)(gl + i);
                a = float4{__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w)};
                *(float4*)(xl + i) = a;
            }
            if (blockIdx.x == 0) {
                if (nrm.x_out) *(float4*)(nrm.x_out + i) = a;
                if (nrm.rec) *(float4*)(nrm.rec + i) = a;
            }
        }
        if (nrm.r) {
            __syncthreads();
            for (size_t c = wave; c * 1024 < xlen; c += 4)
                copy_1k(nrm.gamma, xlen, c * 1024, l8 + xb + c * 1024, lane);
        }
        if (tid < 64) {
            const double ss = rms_sumsq<16>(xl, cols, tid);
            if (tid == 0) nsc = rms_scale(ss, cols, nrm.eps);
        }
        if (nrm.r) wait_vm_keep<0>();  // gamma's copies (the weight groups with them)
        __syncthreads();
        const float sc = nsc;
        for (int i = 4 * tid; i < cols; i += 4 * 256) {
            const float4 a = *(const float4*)(xl + i), g = *(const float4*)(gl + i);
            *(float4*)(xl + i) = float4{__fmul_rn(__fmul_rn(a.x, sc), g.x), __fmul_rn(__fmul_rn(a.y, sc), g.y),
                                        __fmul_rn(__fmul_rn(a.z, sc), g.z), __fmul_rn(__fmul_rn(a.w, sc), g.w)};
        }
        __syncthreads();
        if (DT == 2) {
            // Q4: the block sums of the normed input (scalar.rs:355-359), in
            // gamma's place, for the bias dot.
            for (int b = tid; b < nb; b += 256) gl[b] = m1_block_sum(xl + 32 * b);
            __syncthreads();
        }
    } else {
        // The first weight groups are in flight while x is copied to LDS
        // (indices clamped to the row's last group: a few repeated loads at
        // the row's end are never used).
#pragma unroll
        for (int d = 0; d < PF0; ++d) v2_load<DT, R>(slot[d], qrow, srow, d < ng ? d : ng - 1);
        for (int m = 0; m < M; ++m)
            for (int i = 4 * (int)threadIdx.x; i < cols; i += 4 * 256)
                *(float4*)(xl + m * cols + i) =
                    __builtin_bit_cast(float4, *(const f4u*)(x + (size_t)m * x_stride + i));
        __syncthreads();
    }

    if constexpr (PF == 2) {
        // Two slots: the next group's loads are issued before this group's
        // arithmetic.
        for (int g = 0; g < ng; g += 2) {
            if (g + 1 < ng) v2_load<DT, R>(slot[1], qrow, srow, g + 1);
            v2_group<DT, R, M, false>(acc, slot[0], g, nb, xl, j);
            if (g + 1 >= ng) break;
            if (g + 2 < ng) v2_load<DT, R>(slot[0], qrow, srow, g + 2);
            v2_group<DT, R, M, false>(acc, slot[1], g + 1, nb, xl, j);
        }
    } else {
        // Whole groups in rounds of PF, then the rest (the last group may
        // be partial).
        const int ngf = nb / G;
        int g = 0;
        for (; g + PF <= ngf; g += PF) {
#pragma unroll
            for (int d = 0; d < PF; ++d) {
                v2_group<DT, R, M, true>(acc, slot[d], g + d, nb, xl, j);
                const int gn = g + d + PF;
                v2_load<DT, R>(slot[d], qrow, srow, gn < ng ? gn : ng - 1);
            }
        }
#pragma unroll
        for (int d = 0; d < PF; ++d)
            if (g + d < ng) v2_group<DT, R, M, false>(acc, slot[d], g + d, nb, xl, j);
    }

    uint64_t key = 0;  // this lane's largest argmax key (M = 1, part != nullptr)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const bool valid = (blockIdx.x * R + r) * 32 + lg < rows;
        float bdot[M];
        if (DT == 2) {
            // dot_bf16_f32 (scalar.rs:334-347): lane j runs accumulator lane j
            // over whole groups of 8 blocks, then hsum8 (xor-4, xor-1, xor-2)
            // and the unfused tail.
            const uint16_t* brow = biases + (size_t)row[r] * nb;
            const int body = nb & ~7;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float* xs =
                    NORM ? (const float*)((const unsigned char*)xl + m1x_x_bytes(nb)) : xsum + (size_t)m * nb;
                float a = 0.0f;
                for (int i = j; i < body; i += 8) a = __builtin_fmaf(bf16f(brow[i]), xs[i], a);
                float p = __fadd_rn(a, xor_get(a, 4));
                float q = __fadd_rn(p, xor_get(p, 1));
                float s = __fadd_rn(q, xor_get(q, 2));
                for (int i = body; i < nb; ++i) s = __fadd_rn(s, __fmul_rn(bf16f(brow[i]), xs[i]));
                bdot[m] = s;
            }
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            // Lane p in {0, 1} ends with v[4p + e] in slot e: chains l, 8+l sit
            // in lanes l/4 and l/4 + 2, chains 16+l, 24+l in l/4 + 4 and l/4 + 6.
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float t = __fadd_rn(acc[r][m][e], xor_get(acc[r][m][e], 2));
                v[e] = __fadd_rn(t, xor_get(t, 4));
            }
            float w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = __fadd_rn(v[e], xor_get(v[e], 1));  // v[e] + v[4+e] at lane 0
            float res = __fadd_rn(__fadd_rn(w[0], w[1]), __fadd_rn(w[2], w[3]));
            if (DT == 2) res = __fadd_rn(res, bdot[m]);
            if (valid && j == 0) y[(size_t)m * y_stride + row[r]] = res;
            if (M == 1 && valid && j == 0) {
                const uint64_t k = argmax_key(res, (uint32_t)row[r]);
                key = k > key ? k : key;
            }
        }
    }
    if (M == 1 && part) {
        // The workgroup's largest key (the argmax's first stage, fused).
        __shared__ uint64_t red[4];
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)key, s, 64), hi = __shfl_xor((uint32_t)(key >> 32), s, 64);
            const uint64_t o = ((uint64_t)hi << 32) | lo;
            key = o > key ? o : key;
        }
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = key;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint64_t k = red[0];
            for (int w = 1; w < 4; ++w) k = red[w] > k ? red[w] : k;
            part[blockIdx.x] = k;
        }
    }
}

template <int DT, int M, int R, int PF>
void launch_v2_rp(const uint8_t* fq, const uint16_t* fs, const uint16_t* bi, const float* x, size_t xs,
                  const float* xsum, int rows, int nb, int nbp, float* y, size_t ys, uint64_t* part, hipStream_t st) {
    const dim3 grid(ceil_div(rows, 32 * R)), block(256);
    const size_t lds = (size_t)M * nb * 32 * sizeof(float);
    gemv_f32_v2_kernel<DT, M, R, PF>
        <<<grid, block, lds, st>>>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, part, NormIn{});
}

// One vector with the fused residual add and RMSNorm (x, r and gamma: 16-byte
// aligned, x of at most 64 KB: twice that in LDS).
template <int DT>
void launch_v2_norm(const uint8_t* fq, const uint16_t* fs, const uint16_t* bi, const NormIn& nrm, int rows, int nb,
                    int nbp, float* y, hipStream_t st) {
    static const bool once = [] {
        return hipFuncSetAttribute((const void*)gemv_f32_v2_kernel<DT, 1, 1, 4, true>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 2 * F32_V2_MAX_LDS) == hipSuccess;
    }();
    (void)once;
    const dim3 grid(ceil_div(rows, 32)), block(256);
    const size_t lds = 2 * m1x_x_bytes(nb);  // x, then r / gamma / Q4's block sums
    gemv_f32_v2_kernel<DT, 1, 1, 4, true>
        <<<grid, block, lds, st>>>(fq, fs, bi, nullptr, 0, nullptr, rows, nb, nbp, y, rows, nullptr, nrm);
}

// Rows per lane group: one vector takes one (the most waves; measured
// faster than four at every height up to the vocabulary heads). Several
// vectors take four, so that each x read serves four rows, when that still
// leaves a workgroup per CU (two vectors: four per CU), else one; the
// prefetch depth is four groups for one vector, two for several.
template <int DT, int M>
void launch_v2_m(const uint8_t* fq, const uint16_t* fs, const uint16_t* bi, const float* x, size_t xs,
                 const float* xsum, int rows, int nb, int nbp, float* y, size_t ys, uint64_t* part, hipStream_t st) {
    if constexpr (M == 1)
        launch_v2_rp<DT, 1, 1, 4>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, part, st);
    else if (ceil_div(rows, 32 * V2_R) >= (M == 2 ? 4 : 1) * cu_count())
        launch_v2_rp<DT, M, V2_R, 2>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, part, st);
    else
        launch_v2_rp<DT, M, 1, 2>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, part, st);
}

template <int DT>
void launch_dt_v2(int M, const uint8_t* fq, const uint16_t* fs, const uint16_t* bi, const float* x, size_t xs,
                  const float* xsum, int rows, int nb, int nbp, float* y, size_t ys, hipStream_t st) {
    switch (M) {
        case 1: launch_v2_m<DT, 1>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, nullptr, st); break;
        case 2: launch_v2_m<DT, 2>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, nullptr, st); break;
        case 3: launch_v2_m<DT, 3>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, nullptr, st); break;
        default: launch_v2_m<DT, 4>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys, nullptr, st); break;
    }
}

template <int DT>
void launch_dt(int M, const uint8_t* fq, const uint16_t* fs, const uint16_t* bi, const float* x, size_t xs,
               const float* xsum, int rows, int nb, int nbp, float* y, size_t ys, hipStream_t st) {
    dim3 grid(ceil_div(rows, 16)), block(256);
    switch (M) {
        case 1: gemv_f32_kernel<DT, 1><<<grid, block, 0, st>>>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys); break;
        case 2: gemv_f32_kernel<DT, 2><<<grid, block, 0, st>>>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys); break;
        case 3: gemv_f32_kernel<DT, 3><<<grid, block, 0, st>>>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys); break;
        default: gemv_f32_kernel<DT, 4><<<grid, block, 0, st>>>(fq, fs, bi, x, xs, xsum, rows, nb, nbp, y, ys); break;
    }
}

}  // namespace

size_t f32_quant_bytes(int dtype, int rows, int nb, bool v2) {
    if (!v2) return (size_t)rows * ((nb + (dtype == 1 ? 7 : 15)) / (dtype == 1 ? 8 : 16)) * 256;
    const int g = dtype == 1 ? 4 : 8;
    return (size_t)((rows + 31) / 32) * 32 * ((nb + g - 1) / g) * 128;
}

void launch_relayout_f32(int dtype, const uint8_t* raw_qs, const uint16_t* raw_scales, uint8_t* fq, uint16_t* fs,
                         int rows, int nb, int nbp, bool v2, hipStream_t st) {
    if (v2) {
        const size_t words = f32_quant_bytes(dtype, rows, nb, true) / 4;
        const unsigned blocks = (unsigned)((words + 255) / 256);
        if (dtype == 1)
            relayout_q8_v2_kernel<<<blocks, 256, 0, st>>>(raw_qs, fq, rows, nb);
        else
            relayout_q4_v2_kernel<<<blocks, 256, 0, st>>>(raw_qs, fq, rows, nb);
    } else {
        size_t qbytes = f32_quant_bytes(dtype, rows, nb, false);
        int blocks = (int)((qbytes + 255) / 256);
        if (dtype == 1)
            relayout_q8_kernel<<<blocks, 256, 0, st>>>(raw_qs, fq, rows, nb);
        else
            relayout_q4_kernel<<<blocks, 256, 0, st>>>(raw_qs, fq, rows, nb);
    }
    size_t sn = (size_t)rows * nbp;
    pad_scales_kernel<<<(int)((sn + 255) / 256), 256, 0, st>>>(raw_scales, fs, rows, nb, nbp);
}

void launch_block_sums(const float* x, size_t x_stride, int nb, int n_tok, float* xsum, hipStream_t st) {
    int n = nb * n_tok;
    block_sums_kernel<<<ceil_div(n, 256), 256, 0, st>>>(x, x_stride, nb, n_tok, xsum);
}

// Tokens in chunks of up to four per launch: every token's chains are
// independent, so the chunking never changes a bit.
int f32_v2_parts(int rows) { return ceil_div(rows, 32); }  // one vector: one row per lane group

void launch_gemv_f32_v2_argmax(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases,
                               const float* x, float* xsum, int rows, int nb, int nbp, float* y, uint64_t* part,
                               hipStream_t st) {
    if (dtype == 2) launch_block_sums(x, (size_t)nb * 32, nb, 1, xsum, st);
    if (dtype == 1)
        launch_v2_m<1, 1>(fq, fs, biases, x, (size_t)nb * 32, xsum, rows, nb, nbp, y, rows, part, st);
    else
        launch_v2_m<2, 1>(fq, fs, biases, x, (size_t)nb * 32, xsum, rows, nb, nbp, y, rows, part, st);
}

// The fused residual add and RMSNorm alone (when no fused gemv applies):
// one workgroup, v in LDS (cols floats), the normed input to `out`.
__global__ __launch_bounds__(256) void rmsnorm_vec_kernel(NormIn n, int cols, float* __restrict__ out) {
    extern __shared__ float v[];
    __shared__ float sc;
    const int tid = threadIdx.x;
    for (int i = tid; i < cols; i += 256) {
        float a = n.x[i];
        if (n.r) a = __fadd_rn(a, n.r[i]);
        v[i] = a;
        if (n.x_out) n.x_out[i] = a;
        if (n.rec) n.rec[i] = a;
    }
    __syncthreads();
    if (tid < 64) {
        const double ss = rms_sumsq(v, cols, tid);
        if (tid == 0) sc = rms_scale(ss, cols, n.eps);
    }
    __syncthreads();
    for (int i = tid; i < cols; i += 256) out[i] = __fmul_rn(__fmul_rn(v[i], sc), n.gamma[i]);
}

bool launch_gemv_f32_norm(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases,
                          const NormIn& nrm, int rows, int nb, int nbp, float* y, bool v2, hipStream_t st) {
    const auto a16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    const bool aligned = a16(nrm.x) && a16(nrm.gamma) && (!nrm.r || a16(nrm.r)) && (!nrm.x_out || a16(nrm.x_out)) &&
                         (!nrm.rec || a16(nrm.rec));
    if (!aligned) return false;
    if (v2) {
        if ((size_t)nb * 32 * 4 > (size_t)F32_V2_MAX_LDS) return false;
        if (dtype == 1)
            launch_v2_norm<1>(fq, fs, biases, nrm, rows, nb, nbp, y, st);
        else
            launch_v2_norm<2>(fq, fs, biases, nrm, rows, nb, nbp, y, st);
        return true;
    }
    if (!m1r_fits(dtype, rows, nb, nrm.x)) return false;
    const int nbpq = dtype == 1 ? (nb + 7) / 8 * 8 : (nb + 15) / 16 * 16;
    if (m1x_lds(dtype, nb, nbpq, 8, true) > M1R_MAX_LDS) return false;
    const F32Mat m{fq, fs, biases, rows, nb, nbp};
    if (dtype == 1)
        launch_m1x<1, true>(m, nullptr, y, nrm, st);
    else
        launch_m1x<2, true>(m, nullptr, y, nrm, st);
    return true;
}

void launch_rmsnorm_vec(const NormIn& nrm, int cols, float* out, hipStream_t st) {
    static const bool once = [] {
        return hipFuncSetAttribute((const void*)rmsnorm_vec_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)(64 * 1024)) == hipSuccess;
    }();
    (void)once;
    rmsnorm_vec_kernel<<<1, 256, (size_t)cols * 4, st>>>(nrm, cols, out);
}

void launch_gemv_f32(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases, const float* x,
                     size_t x_stride, float* xsum, int rows, int nb, int nbp, int n_tok, float* y,
                     size_t y_stride, bool v2, hipStream_t st) {
    // Q4 block sums, except for the one-vector kernel, which forms its own.
    const auto one = [&](const float* xt) { return !v2 && (nb <= M1_MAX_NB || m1r_fits(dtype, rows, nb, xt)); };
    // Several vectors on the 16-lane layout: the one-vector kernels once
    // per vector, which stage x in LDS and keep weight groups in flight
    // (the several-vector kernel reads x from global memory at every
    // block). Measured faster for Q8 at every shape (2-9x) and for Q4 from
    // 64 blocks; each vector's chains are independent, so the bits are the
    // same either way.
    if (n_tok > 1 && !v2 && (dtype == 1 || nb >= M1W_MIN_NB)) {
        bool all = true;
        for (int t = 0; t < n_tok && all; ++t) all = one(x + (size_t)t * x_stride);
        if (all) {
            for (int t = 0; t < n_tok; ++t) {
                if (dtype == 1)
                    launch_m1<1>(fq, fs, biases, x + (size_t)t * x_stride, rows, nb, nbp, y + (size_t)t * y_stride, st);
                else
                    launch_m1<2>(fq, fs, biases, x + (size_t)t * x_stride, rows, nb, nbp, y + (size_t)t * y_stride, st);
            }
            return;
        }
    }
    if (dtype == 2 && !(n_tok == 1 && one(x))) launch_block_sums(x, x_stride, nb, n_tok, xsum, st);
    // The 8-lane kernel keeps x in LDS: at most 64 KB of it per launch.
    int per = 4;
    if (v2 && per * nb * 32 * 4 > F32_V2_MAX_LDS) per = F32_V2_MAX_LDS / (nb * 32 * 4);
    for (int t0 = 0; t0 < n_tok; t0 += per) {
        int m = n_tok - t0 < per ? n_tok - t0 : per;
        const float* xt = x + (size_t)t0 * x_stride;
        const float* st_xsum = xsum ? xsum + (size_t)t0 * nb : nullptr;
        float* yt = y + (size_t)t0 * y_stride;
        if (m == 1 && one(xt)) {
            if (dtype == 1)
                launch_m1<1>(fq, fs, biases, xt, rows, nb, nbp, yt, st);
            else
                launch_m1<2>(fq, fs, biases, xt, rows, nb, nbp, yt, st);
        } else if (v2) {
            if (dtype == 1)
                launch_dt_v2<1>(m, fq, fs, biases, xt, x_stride, st_xsum, rows, nb, nbp, yt, y_stride, st);
            else
                launch_dt_v2<2>(m, fq, fs, biases, xt, x_stride, st_xsum, rows, nb, nbp, yt, y_stride, st);
        } else if (dtype == 1) {
            launch_dt<1>(m, fq, fs, biases, xt, x_stride, st_xsum, rows, nb, nbp, yt, y_stride, st);
        } else {
            launch_dt<2>(m, fq, fs, biases, xt, x_stride, st_xsum, rows, nb, nbp, yt, y_stride, st);
        }
    }
}

}  // namespace nnh
