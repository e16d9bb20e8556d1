// The bit-exact f32 gemv of ONE vector over the 16-lane quant layout, with x
// in LDS: the core of the library's M = 1 kernels and of the fused kernels
// of the device-resident Gemma-3 decode step.
//
// Arithmetic: exactly gemv_f32_kernel's (crates/nncpu/src/kernels/scalar.rs:
// 626-742): chain j of a row (element j of every 32-block) runs over the
// blocks in order, acc = fma(f32(q) * bf16(s), x, acc), then the reduction
// v[l] = (acc_l + acc_{8+l}) + (acc_{16+l} + acc_{24+l}), hsum8, plus the Q4
// bias dot (scalar.rs:334-347).
//
// Schedule: every lane issues all of its row's weight groups at once (one
// 16-byte load per group: Q8 groups of 8 blocks, Q4 groups of 16), and x
// and the scales are read from LDS, whose reads wait on their own counter,
// so they never wait behind a weight load. A caller issues its own global
// loads (x, the scale rows, a fused prologue's inputs) BEFORE prefetch(), so
// that waiting for them does not wait for the weights, fills LDS, then calls
// run().
#pragma once
#include "common.h"

namespace nnh {

constexpr int M1_ROWS = 16;  // rows per 256-thread workgroup, 16 lanes per row

__device__ __forceinline__ uint32_t byte_of(const uint4& v, int i) {
    uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return (w >> (8 * (i & 3))) & 0xffu;
}

__device__ __forceinline__ uint32_t half_of(const uint4& v, int i) {
    uint32_t w = i < 2 ? v.x : i < 4 ? v.y : i < 6 ? v.z : v.w;
    return (w >> (16 * (i & 1))) & 0xffffu;
}

// Wait for this thread's LDS writes, then the workgroup barrier. Unlike
// __syncthreads it leaves vector-memory loads (the weights) in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One matrix in the 16-lane layout of kernels_f32.hip: rows of ngp whole
// groups (Q8: 8 blocks, Q4: 16; the last one zero-filled past nb) of 256
// bytes, one 16-byte piece per lane.
struct F32Mat {
    const uint8_t* fq;   // per-lane quant groups
    const uint16_t* fs;  // scales, rows padded to nbp = ngp * group
    const uint16_t* bi;  // Q4 biases [rows][nb], else null
    int rows, nb, nbp;
};

__device__ __forceinline__ int m1_groups(int dt, int nb) { return dt == 1 ? (nb + 7) / 8 : (nb + 15) / 16; }

// The scale rows row0 .. row0 + nrows - 1 of a matrix, staged into LDS by a
// workgroup of NT threads (MAXB: most bytes staged): load() issues the loads
// (unconditional, clamped, so the caller's wait counts stay exact), store()
// writes them to sl.
template <int NT, int MAXB>
struct ScaleStage {
    static constexpr int K = (MAXB + NT * 16 - 1) / (NT * 16);  // 16-byte pieces per thread
    uint4 v[K];
    int n;
    __device__ __forceinline__ void load(const F32Mat& m, int row0, int nrows) {
        n = nrows * m.nbp / 8;
        const uint16_t* base = m.fs + (size_t)row0 * m.nbp;
#pragma unroll
        for (int k = 0; k < K; ++k) v[k] = *(const uint4*)(base + 8 * min((int)threadIdx.x + NT * k, n - 1));
    }
    __device__ __forceinline__ void store(uint16_t* sl) const {
#pragma unroll
        for (int k = 0; k < K; ++k) *(uint4*)(sl + 8 * min((int)threadIdx.x + NT * k, n - 1)) = v[k];
    }
};

// 16 lanes per row, lane j running chains j and j + 16. D >= the row's
// groups: every group is in flight from prefetch() on (slots past the last
// group reload it), and prefetch() is unconditional, so the compiler's wait
// counts before the caller's first barrier are exact and never wait for
// the weights.
template <int DT, int D>
struct M1Lane {
    static constexpr int G = DT == 1 ? 8 : 16;  // blocks per group

    const uint8_t* qrow;
    int nb, ngp, j;
    uint4 q[D];
    float a0, a1;

    __device__ __forceinline__ void init(const F32Mat& m, int row, int lane) {
        nb = m.nb;
        ngp = m1_groups(DT, nb);
        j = lane;
        qrow = m.fq + (size_t)row * ngp * 256;
        a0 = a1 = 0.0f;
    }

    __device__ __forceinline__ void prefetch() {
#pragma unroll
        for (int d = 0; d < D; ++d) q[d] = load_nt16u(qrow + (size_t)(d < ngp ? d : ngp - 1) * 256 + j * 16);
    }

    __device__ __forceinline__ void block(uint32_t qq, float s_b, float x0, float x1) {
        float w0, w1;
        if (DT == 1) {
            w0 = (float)(int8_t)(qq & 0xffu) * s_b;  // exact
            w1 = (float)(int8_t)(qq >> 8) * s_b;
        } else {
            w0 = (float)(qq & 15u) * s_b;
            w1 = (float)(qq >> 4) * s_b;
        }
        a0 = __builtin_fmaf(w0, x0, a0);
        a1 = __builtin_fmaf(w1, x1, a1);
    }

    // Blocks gG .. gG + nblk - 1 (FULL: nblk = G; else the partial last
    // group); the group's x values and scales are read from LDS first.
    template <bool FULL>
    __device__ __forceinline__ void group(const uint4& qv, int g, int nblk, const float* xl, const uint16_t* sl) {
        const float* xb = xl + 32 * g * G + j;
        uint4 sv[G / 8];
#pragma unroll
        for (int k = 0; k < G / 8; ++k) sv[k] = *(const uint4*)(sl + g * G + 8 * k);
        float x0[G], x1[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            x0[i] = FULL || i < nblk ? xb[32 * i] : 0.0f;
            x1[i] = FULL || i < nblk ? xb[32 * i + 16] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
            if (FULL || i < nblk) {
                const float sb = bf16f(half_of(sv[i / 8], i % 8));
                const uint32_t qq = DT == 1 ? (byte_of(qv, 2 * i) | byte_of(qv, 2 * i + 1) << 8) : byte_of(qv, i);
                block(qq, sb, x0[i], x1[i]);
            }
        }
    }

    // All blocks, in order. xl: x of the row's columns in LDS; sl: the row's
    // padded scale row in LDS.
    __device__ __forceinline__ void run(const float* xl, const uint16_t* sl) {
        const int ng = nb / G;  // whole groups; a partial one follows when nb % G
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (d < ng)
                group<true>(q[d], d, G, xl, sl);
            else if (d == ng && d < ngp)
                group<false>(q[d], d, nb - d * G, xl, sl);
        }
    }

    // The row's sum (valid at lane j == 0 of the row's 16): v[l] = (acc_l +
    // acc_{8+l}) + (acc_{16+l} + acc_{24+l}) by xor-8, then hsum8 by xor-4,
    // xor-1, xor-2.
    __device__ __forceinline__ float reduce() const {
        const float u = __fadd_rn(a0, xor_get(a0, 8));
        const float w = __fadd_rn(a1, xor_get(a1, 8));
        const float v = __fadd_rn(u, w);
        const float p = __fadd_rn(v, xor_get(v, 4));
        const float qq = __fadd_rn(p, xor_get(p, 1));
        return __fadd_rn(qq, xor_get(qq, 2));
    }
};

// The wide mapping for long rows: 32 lanes per row, lane j running chain j
// alone. It reads the same 16-lane layout: lanes j and j + 16 load the same
// 16-byte piece (j mod 16) and take its even / odd bytes (Q8: elements j,
// j + 16 of each block) or its low / high nibbles (Q4). As M1Lane, every
// group is in flight from prefetch() on and the scales come from LDS; x
// from a transposed LDS copy (m1w_xpos), so a lane's x values for 8 blocks
// are two 16-byte reads. Reduction: xor-8, xor-16 give v[l] at lane l < 8,
// then hsum8 (xor-4, xor-1, xor-2): the same additions.
__device__ __forceinline__ int m1w_stride(int nb) {
    const int s = (nb + 3) & ~3;  // 16-byte rows; an odd number of 16-byte units spreads the banks
    return (s & 4) ? s : s + 4;
}
inline int m1w_stride_host(int nb) {
    const int s = (nb + 3) & ~3;
    return (s & 4) ? s : s + 4;
}
// Position of x[32 b + c] in the transposed copy.
__device__ __forceinline__ int m1w_xpos(int b, int c, int S) { return c * S + b; }

template <int DT, int D>
struct M1Wide {
    static constexpr int G = DT == 1 ? 8 : 16;

    const uint8_t* qrow;
    int nb, ngp, j, pj, h, S;
    uint4 q[D];
    float a;

    __device__ __forceinline__ void init(const F32Mat& m, int row, int lane) {
        nb = m.nb;
        ngp = m1_groups(DT, nb);
        j = lane;
        pj = lane & 15;
        h = lane >> 4;
        S = m1w_stride(nb);
        qrow = m.fq + (size_t)row * ngp * 256;
        a = 0.0f;
    }

    __device__ __forceinline__ void prefetch() {
#pragma unroll
        for (int d = 0; d < D; ++d) q[d] = load_nt16u(qrow + (size_t)(d < ngp ? d : ngp - 1) * 256 + pj * 16);
    }

    // The lane's weight of a block: Q8 byte h of the pair, Q4 nibble h.
    __device__ __forceinline__ float weight(uint32_t qq, float sb) const {
        if (DT == 1) return (float)(int8_t)((qq >> (8 * h)) & 0xffu) * sb;
        return (float)((qq >> (4 * h)) & 15u) * sb;
    }

    template <bool FULL>
    __device__ __forceinline__ void group(const uint4& qv, int g, int nblk, const float* xw, const uint16_t* sl) {
        const float* xp = xw + j * S + g * G;
        float x[G];
        uint4 sv[G / 8];
#pragma unroll
        for (int k = 0; k < G / 8; ++k) sv[k] = *(const uint4*)(sl + g * G + 8 * k);
#pragma unroll
        for (int i = 0; i < G; i += 4) {
            if (FULL || i < nblk) {
                const float4 v = *(const float4*)(xp + i);
                x[i] = v.x;
                x[i + 1] = v.y;
                x[i + 2] = v.z;
                x[i + 3] = v.w;
            } else {
                x[i] = x[i + 1] = x[i + 2] = x[i + 3] = 0.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
            if (FULL || i < nblk) {
                const uint32_t qq = DT == 1 ? (byte_of(qv, 2 * i) | byte_of(qv, 2 * i + 1) << 8) : byte_of(qv, i);
                a = __builtin_fmaf(weight(qq, bf16f(half_of(sv[i / 8], i % 8))), x[i], a);
            }
        }
    }

    __device__ __forceinline__ void run(const float* xw, const uint16_t* sl) {
        const int ng = nb / G;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (d < ng)
                group<true>(q[d], d, G, xw, sl);
            else if (d == ng && d < ngp)
                group<false>(q[d], d, nb - d * G, xw, sl);
        }
    }

    __device__ __forceinline__ float reduce() const {
        const float u = __fadd_rn(a, xor_get(a, 8));
        const float v = __fadd_rn(u, xor_get(u, 16));
        const float p = __fadd_rn(v, xor_get(v, 4));
        const float qq = __fadd_rn(p, xor_get(p, 1));
        return __fadd_rn(qq, xor_get(qq, 2));
    }
};

// Q4 bias term of one row, dot_bf16_f32 (scalar.rs:334-347): lanes 0..7 of
// the row's lanes run the 8 accumulator lanes over whole groups of 8
// blocks, hsum8 (xor-4, xor-1, xor-2), then the unfused tail. bl: the row's
// biases, xs: the block sums of x. Valid at lane 0.
__device__ __forceinline__ float m1_bias_dot(const uint16_t* bl, const float* xs, int nb, int j) {
    const int body = nb & ~7;
    float a = 0.0f;
    if (j < 8)
        for (int i = j; i < body; i += 8) a = __builtin_fmaf(bf16f(bl[i]), xs[i], a);
    const float p = __fadd_rn(a, xor_get(a, 4));
    const float q = __fadd_rn(p, xor_get(p, 1));
    float s = __fadd_rn(q, xor_get(q, 2));
    for (int i = body; i < nb; ++i) s = __fadd_rn(s, __fmul_rn(bf16f(bl[i]), xs[i]));
    return s;
}

// Block sum of x (scalar.rs:355-359): hsum8 of ((c[l]+c[8+l])+c[16+l])+c[24+l].
__device__ __forceinline__ float m1_block_sum(const float* c) {
    float v[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) v[l] = __fadd_rn(__fadd_rn(__fadd_rn(c[l], c[8 + l]), c[16 + l]), c[24 + l]);
    return __fadd_rn(__fadd_rn(__fadd_rn(v[0], v[4]), __fadd_rn(v[1], v[5])),
                     __fadd_rn(__fadd_rn(v[2], v[6]), __fadd_rn(v[3], v[7])));
}

}  // namespace nnh
