// The bit-exact f32 gemv of ONE vector over the 16-lane quant layout, with x
// in LDS: the core of the library's M = 1 kernel and of the fused kernels of
// the device-resident Gemma-3 decode step.
//
// Arithmetic: exactly gemv_f32_kernel's (crates/nncpu/src/kernels/scalar.rs:
// 626-742): lane j of a row's 16 runs chains j and j + 16 over the blocks in
// order, acc = fma(f32(q) * bf16(s), x, acc), then the xor-8 / 4 / 1 / 2
// reduction tree, plus the Q4 bias dot (scalar.rs:334-347).
//
// Schedule: every lane keeps a ring of D weight groups in flight (Q8 groups
// of 8 blocks, Q4 groups of 16), refilling a slot as soon as its group is
// consumed; x is read from LDS, whose reads wait on their own
// counter, so an x read never waits behind a weight load. A caller issues its
// own global loads (x, or a fused prologue's inputs) BEFORE prefetch(), so
// that waiting for them does not wait for the ring, fills LDS, then calls
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
// __syncthreads it leaves vector-memory loads (the weight ring) in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One matrix in the 16-lane layout of kernels_f32.hip.
struct F32Mat {
    const uint8_t* fq;   // per-lane quant groups
    const uint16_t* fs;  // scales, rows padded to nbp
    const uint16_t* bi;  // Q4 biases [rows][nb], else null
    int rows, nb, nbp;
};

// D: groups in the ring. Everything prefetch() issues is unconditional (a
// group index past the last whole group is clamped to the last one, or to 0
// when there is none: the quant allocation has 256 spare bytes for that), so
// the compiler's wait counts before the caller's first barrier are exact and
// never wait for the ring.
template <int DT, int D>
struct M1Lane {
    static constexpr int G = DT == 1 ? 8 : 16;  // blocks per group
    static constexpr int SW = DT == 1 ? 1 : 2;  // 16-byte scale loads per group

    const uint8_t* qrow;
    const uint16_t* srow;
    int nb, ng, t, j;
    uint4 q[D], s[D][SW];
    uint32_t tq[G - 1];  // tail quants: Q8 one 16-bit pair per block, Q4 one byte
    uint4 ts[SW];
    float a0, a1;

    __device__ __forceinline__ void init(const F32Mat& m, int row, int lane) {
        nb = m.nb;
        ng = nb / G;
        t = nb - ng * G;
        j = lane;
        qrow = m.fq + (size_t)row * nb * (DT == 1 ? 32 : 16);
        srow = m.fs + (size_t)row * m.nbp;
        a0 = a1 = 0.0f;
    }

    __device__ __forceinline__ void load(int slot, int g) {
        q[slot] = load_nt16u(qrow + (size_t)g * 256 + j * 16);
#pragma unroll
        for (int k = 0; k < SW; ++k) s[slot][k] = *(const uint4*)(srow + g * G + 8 * k);
    }

    // The tail (one load per block slot, from the row's start when unused)
    // and the ring's first D groups.
    __device__ __forceinline__ void prefetch() {
        const uint8_t* tp = qrow + (size_t)ng * 256 + (size_t)j * (DT == 1 ? 2 : 1) * t;
#pragma unroll
        for (int i = 0; i < G - 1; ++i)
            tq[i] = DT == 1 ? (uint32_t)*(const uint16_t*)(i < t ? tp + 2 * i : qrow)
                            : (uint32_t)*(i < t ? tp + i : qrow);
#pragma unroll
        for (int k = 0; k < SW; ++k) ts[k] = *(const uint4*)(srow + (t ? ng * G : 0) + 8 * k);
        const int last = ng > 0 ? ng - 1 : 0;
#pragma unroll
        for (int d = 0; d < D; ++d) load(d, d < ng ? d : last);
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

    // One group: its x values are read from LDS first, all together.
    __device__ __forceinline__ void group(const uint4& qv, const uint4 (&sv)[SW], int g, const float* xl) {
        const float* xb = xl + 32 * g * G + j;
        float x0[G], x1[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
            x0[i] = xb[32 * i];
            x1[i] = xb[32 * i + 16];
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const float sb = bf16f(half_of(sv[i / 8], i % 8));
            const uint32_t qq = DT == 1 ? (byte_of(qv, 2 * i) | byte_of(qv, 2 * i + 1) << 8) : byte_of(qv, i);
            block(qq, sb, x0[i], x1[i]);
        }
    }

    // All blocks, in order. xl: x of the row's columns, in LDS. A slot is
    // refilled right after its group is used, in the same registers, so the
    // loop carries no copies of in-flight values (a copy would wait for them).
    __device__ __forceinline__ void run(const float* xl) {
        int g0 = 0;
        for (; g0 + 2 * D <= ng; g0 += D) {  // every refill in range
#pragma unroll
            for (int d = 0; d < D; ++d) {
                group(q[d], s[d], g0 + d, xl);
                __builtin_amdgcn_sched_barrier(0);  // the refill stays after the use
                load(d, g0 + d + D);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (g0 + d < ng) {
                group(q[d], s[d], g0 + d, xl);
                __builtin_amdgcn_sched_barrier(0);
                if (g0 + d + D < ng) load(d, g0 + d + D);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (g0 + D + d < ng) group(q[d], s[d], g0 + D + d, xl);
        const float* xt = xl + 32 * ng * G + j;
#pragma unroll
        for (int i = 0; i < G - 1; ++i)
            if (i < t) block(tq[i], bf16f(half_of(ts[i / 8], i % 8)), xt[32 * i], xt[32 * i + 16]);
    }

    // The row's sum (valid at lane j == 0 of the row's 16): v[l] = (acc_l +
    // acc_{8+l}) + (acc_{16+l} + acc_{24+l}), then hsum8.
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
// alone, 8 rows per 256-thread workgroup. It reads the same 16-lane layout:
// lanes j and j + 16 load the same 16-byte piece (j mod 16) and take its
// even / odd bytes (Q8: elements j, j + 16 of each block) or its low / high
// nibbles (Q4). The whole row is in flight at once: the ring has a slot for
// every group (D >= the row's groups) and holds quants only; the scales are
// read from an LDS copy of the workgroup's scale rows, x from a transposed
// LDS copy (m1w_xpos), so a lane's x values for 8 blocks are two 16-byte
// reads. Reduction: xor-8, xor-16 give v[l] at lane l < 8, then hsum8
// (xor-4, xor-1, xor-2): the same additions.
__device__ __forceinline__ int m1w_stride(int nb) {
    const int s = (nb + 3) & ~3;  // 16-byte rows; an odd number of 16-byte units spreads the banks
    return (s & 4) ? s : s + 4;
}
// Position of x[32 b + c] in the transposed copy.
__device__ __forceinline__ int m1w_xpos(int b, int c, int S) { return c * S + b; }

template <int DT, int D>
struct M1Wide {
    static constexpr int G = DT == 1 ? 8 : 16;

    const uint8_t* qrow;
    int nb, ng, t, j, pj, h, S;
    uint4 q[D];
    uint32_t tq[G - 1];
    float a;

    __device__ __forceinline__ void init(const F32Mat& m, int row, int lane) {
        nb = m.nb;
        ng = nb / G;
        t = nb - ng * G;
        j = lane;
        pj = lane & 15;
        h = lane >> 4;
        S = m1w_stride(nb);
        qrow = m.fq + (size_t)row * nb * (DT == 1 ? 32 : 16);
        a = 0.0f;
    }

    // The tail and every group (D >= ng; slots past the last group reload
    // it), all unconditional, so waits before the caller's first barrier are
    // exact.
    __device__ __forceinline__ void prefetch() {
        const uint8_t* tp = qrow + (size_t)ng * 256 + (size_t)pj * (DT == 1 ? 2 : 1) * t;
#pragma unroll
        for (int i = 0; i < G - 1; ++i)
            tq[i] = DT == 1 ? (uint32_t)*(const uint16_t*)(i < t ? tp + 2 * i : qrow)
                            : (uint32_t)*(i < t ? tp + i : qrow);
        const int last = ng > 0 ? ng - 1 : 0;
#pragma unroll
        for (int d = 0; d < D; ++d) q[d] = load_nt16u(qrow + (size_t)(d < ng ? d : last) * 256 + pj * 16);
    }

    // The lane's weight of block i of a group: Q8 byte 2i + h, Q4 nibble h of byte i.
    __device__ __forceinline__ float weight(uint32_t qq, float sb) const {
        if (DT == 1) return (float)(int8_t)((qq >> (8 * h)) & 0xffu) * sb;
        return (float)((qq >> (4 * h)) & 15u) * sb;
    }

    // sl: the row's scales in LDS.
    __device__ __forceinline__ void group(const uint4& qv, int g, const float* xw, const uint16_t* sl) {
        const float* xp = xw + j * S + g * G;
        float x[G];
        uint4 sv[G / 8];
#pragma unroll
        for (int k = 0; k < G / 8; ++k) sv[k] = *(const uint4*)(sl + g * G + 8 * k);
#pragma unroll
        for (int i = 0; i < G; i += 4) {
            const float4 v = *(const float4*)(xp + i);
            x[i] = v.x;
            x[i + 1] = v.y;
            x[i + 2] = v.z;
            x[i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
            const uint32_t qq = DT == 1 ? (byte_of(qv, 2 * i) | byte_of(qv, 2 * i + 1) << 8) : byte_of(qv, i);
            a = __builtin_fmaf(weight(qq, bf16f(half_of(sv[i / 8], i % 8))), x[i], a);
        }
    }

    __device__ __forceinline__ void run(const float* xw, const uint16_t* sl) {
#pragma unroll
        for (int d = 0; d < D; ++d)
            if (d < ng) group(q[d], d, xw, sl);
        const float* xt = xw + j * S + ng * G;
#pragma unroll
        for (int i = 0; i < G - 1; ++i)
            if (i < t) a = __builtin_fmaf(weight(tq[i], bf16f(sl[ng * G + i])), xt[i], a);
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
// the row's 16 run the 8 accumulator lanes over whole groups of 8 blocks,
// hsum8 (xor-4, xor-1, xor-2), then the unfused tail. bl: the row's biases,
// xs: the block sums of x. Valid at lane 0.
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
