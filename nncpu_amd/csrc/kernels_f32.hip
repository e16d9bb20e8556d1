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
//         q[b0+i][j], q[b0+i][j+16]. A tail of t < 8 blocks gives each lane
//         2t bytes at offset 2t*j.
//   Q4:   groups of 16 blocks; lane j's 16 bytes are byte j of blocks
//         b0..b0+15 (low nibble = chain j, high = chain j+16). A tail of
//         t < 16 blocks gives each lane t bytes at offset t*j.
// Scales are copied to rows padded to nbp (a multiple of 8 / 16) so a
// group's scales are one aligned 16-byte load per 8.

#include "common.h"

namespace nnh {
namespace {

constexpr int Q8_GROUP = 8;
constexpr int Q4_GROUP = 16;

// One thread per source quant byte: raw split layout -> per-lane groups.
__global__ void relayout_q8_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ fq, int rows, int nb) {
    size_t row_bytes = (size_t)nb * 32;
    size_t total = (size_t)rows * row_bytes;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    size_t r = idx / row_bytes;
    int within = (int)(idx - r * row_bytes);
    int b = within >> 5, k = within & 31;
    int j = k & 15, h = k >> 4;
    int ng = nb / Q8_GROUP;
    int g = b / Q8_GROUP;
    size_t off;
    if (g < ng) {
        int i = b - g * Q8_GROUP;
        off = (size_t)g * 256 + j * 16 + 2 * i + h;
    } else {
        int t = nb - ng * Q8_GROUP;
        int i = b - ng * Q8_GROUP;
        off = (size_t)ng * 256 + (size_t)j * 2 * t + 2 * i + h;
    }
    fq[r * row_bytes + off] = raw[idx];
}

__global__ void relayout_q4_kernel(const uint8_t* __restrict__ raw, uint8_t* __restrict__ fq, int rows, int nb) {
    size_t row_bytes = (size_t)nb * 16;
    size_t total = (size_t)rows * row_bytes;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    size_t r = idx / row_bytes;
    int within = (int)(idx - r * row_bytes);
    int b = within >> 4, j = within & 15;
    int ng = nb / Q4_GROUP;
    int g = b / Q4_GROUP;
    size_t off;
    if (g < ng) {
        off = (size_t)g * 256 + j * 16 + (b - g * Q4_GROUP);
    } else {
        int t = nb - ng * Q4_GROUP;
        off = (size_t)ng * 256 + (size_t)j * t + (b - ng * Q4_GROUP);
    }
    fq[r * row_bytes + off] = raw[idx];
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

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xffu;
}

__device__ __forceinline__ uint32_t half_of(const uint4& v, int i) {
    uint32_t w = i < 2 ? v.x : i < 4 ? v.y : i < 6 ? v.z : v.w;
    return (w >> (16 * (i & 1))) & 0xffffu;
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
        const uint8_t* qrow = fq + (size_t)row * nb * 32;
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
        const int t = nb - ng * Q8_GROUP;
        const uint8_t* tq = qrow + (size_t)ng * 256 + (size_t)j * 2 * t;
        for (int i = 0; i < t; ++i) {
            int b = ng * Q8_GROUP + i;
            float s = bf16f(srow[b]);
            float w0 = (float)(int8_t)tq[2 * i] * s;
            float w1 = (float)(int8_t)tq[2 * i + 1] * s;
            step<M>(a0, a1, w0, w1, x, x_stride, (size_t)32 * b + j);
        }
    } else {
        const uint8_t* qrow = fq + (size_t)row * nb * 16;
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
        const uint8_t* tq = qrow + (size_t)ng * 256 + (size_t)j * t;
        for (int i = 0; i < t; ++i) {
            int b = ng * Q4_GROUP + i;
            float s = bf16f(srow[b]);
            uint32_t byte = tq[i];
            float w0 = (float)(byte & 15u) * s;
            float w1 = (float)(byte >> 4) * s;
            step<M>(a0, a1, w0, w1, x, x_stride, (size_t)32 * b + j);
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

void launch_relayout_f32(int dtype, const uint8_t* raw_qs, const uint16_t* raw_scales, uint8_t* fq, uint16_t* fs,
                         int rows, int nb, int nbp, hipStream_t st) {
    size_t qbytes = (size_t)rows * nb * (dtype == 1 ? 32 : 16);
    int blocks = (int)((qbytes + 255) / 256);
    if (dtype == 1)
        relayout_q8_kernel<<<blocks, 256, 0, st>>>(raw_qs, fq, rows, nb);
    else
        relayout_q4_kernel<<<blocks, 256, 0, st>>>(raw_qs, fq, rows, nb);
    size_t sn = (size_t)rows * nbp;
    pad_scales_kernel<<<(int)((sn + 255) / 256), 256, 0, st>>>(raw_scales, fs, rows, nb, nbp);
}

void launch_block_sums(const float* x, size_t x_stride, int nb, int n_tok, float* xsum, hipStream_t st) {
    int n = nb * n_tok;
    block_sums_kernel<<<ceil_div(n, 256), 256, 0, st>>>(x, x_stride, nb, n_tok, xsum);
}

// Tokens in chunks of up to four per launch: every token's chains are
// independent, so the chunking never changes a bit.
void launch_gemv_f32(int dtype, const uint8_t* fq, const uint16_t* fs, const uint16_t* biases, const float* x,
                     size_t x_stride, const float* xsum, int rows, int nb, int nbp, int n_tok, float* y,
                     size_t y_stride, hipStream_t st) {
    for (int t0 = 0; t0 < n_tok; t0 += 4) {
        int m = n_tok - t0 < 4 ? n_tok - t0 : 4;
        const float* xt = x + (size_t)t0 * x_stride;
        const float* st_xsum = xsum ? xsum + (size_t)t0 * nb : nullptr;
        float* yt = y + (size_t)t0 * y_stride;
        if (dtype == 1)
            launch_dt<1>(m, fq, fs, biases, xt, x_stride, st_xsum, rows, nb, nbp, yt, y_stride, st);
        else
            launch_dt<2>(m, fq, fs, biases, xt, x_stride, st_xsum, rows, nb, nbp, yt, y_stride, st);
    }
}

}  // namespace nnh
