// The int8-activation path: activations quantized on the device with nncpu's
// own Q8_0 encoder (crates/nncpu/src/kernels/quant.rs:31-60), exact int32
// block dot products against the weights' integer quants, and the block
// terms scaled and summed in f64.
//
// For a row r and activation vector x' = q_x * s_x (exact in f32), nncpu's
// gemv computes sum_b s_w[r,b] * sum_k q_w[r,32b+k] * x'[32b+k] (+ for Q4
// sum_b bias[r,b] * xsum[b], kernels/mod.rs:848-856). With
// P_b = sum_k q_w * q_x (an exact int32, |P_b| < 2^20) that is
//     y_r = sum_b s_w s_x P_b  (+ bias s_x sum_k q_x),
// each term exact in f64 (at most 8+8+20 significant bits). Summing those in
// f64 and rounding once gives the f32 nearest the exact product of the
// dequantized operands, to within f64 rounding.

#include "common.h"
#include "q8_act.h"
#include "rmsnorm_exact.h"

namespace nnh {
namespace {

// ---- activation quantizer: quant.rs:31-60 on the device ----------------------

// One 32-lane half-wave per block of 32 values.
__global__ __launch_bounds__(256) void quantize_act_kernel(const float* __restrict__ x, size_t x_stride, int cols,
                                                           int n_tok, int8_t* __restrict__ q,
                                                           uint16_t* __restrict__ s, double* __restrict__ sx,
                                                           float* __restrict__ sxT, int tok_pad) {
    const int nb = cols >> 5;
    const int k = threadIdx.x & 31;
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const bool valid = blk < nb * n_tok;
    const int bb = valid ? blk : 0;
    const int t = bb / nb, b = bb - t * nb;
    float v = x[(size_t)t * x_stride + 32 * (size_t)b + k];
    float a = q8_abs(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m, 32));
    const Q8Scale qs = q8_scale(a);
    const uint32_t sbits = qs.bits;
    const float scale = qs.scale;
    const int qi = q8_quant(v, qs.inv);
    int qsum = qi;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) qsum += __shfl_xor(qsum, m, 32);
    if (!valid) return;
    q[(size_t)t * cols + 32 * (size_t)b + k] = (int8_t)qi;
    if (k == 0) {
        s[(size_t)t * nb + b] = (uint16_t)sbits;
        sx[2 * ((size_t)t * nb + b)] = (double)scale;
        sx[2 * ((size_t)t * nb + b) + 1] = (double)scale * (double)qsum;  // exact: s_x * sum(q_x)
        // Block-major f32 copies for the GEMM: [b][tok_pad] scale, then [b][tok_pad] scale * sum(q).
        if (sxT) {
            sxT[(size_t)b * tok_pad + t] = scale;
            sxT[(size_t)nb * tok_pad + (size_t)b * tok_pad + t] = scale * (float)qsum;  // exact: 8 + 13 bits
        }
    }
}

// ---- exact block dots ----------------------------------------------------------

// Q8_0: 32 signed weight bytes against 32 activation bytes.
__device__ __forceinline__ int dot_q8(const int4& w0, const int4& w1, const int4& x0, const int4& x1) {
    int p = 0;
    p = __builtin_amdgcn_sdot4(w0.x, x0.x, p, false);
    p = __builtin_amdgcn_sdot4(w0.y, x0.y, p, false);
    p = __builtin_amdgcn_sdot4(w0.z, x0.z, p, false);
    p = __builtin_amdgcn_sdot4(w0.w, x0.w, p, false);
    p = __builtin_amdgcn_sdot4(w1.x, x1.x, p, false);
    p = __builtin_amdgcn_sdot4(w1.y, x1.y, p, false);
    p = __builtin_amdgcn_sdot4(w1.z, x1.z, p, false);
    p = __builtin_amdgcn_sdot4(w1.w, x1.w, p, false);
    return p;
}

// Q4: byte i of the 16 holds element i (low nibble) and i+16 (high). The
// nibbles are 0..15, so as bytes they are valid non-negative int8 lanes.
__device__ __forceinline__ int dot_q4(const int4& w, const int4& x0, const int4& x1) {
    const int m = 0x0f0f0f0f;
    int p = 0;
    p = __builtin_amdgcn_sdot4(w.x & m, x0.x, p, false);
    p = __builtin_amdgcn_sdot4(w.y & m, x0.y, p, false);
    p = __builtin_amdgcn_sdot4(w.z & m, x0.z, p, false);
    p = __builtin_amdgcn_sdot4(w.w & m, x0.w, p, false);
    p = __builtin_amdgcn_sdot4((int)((unsigned)w.x >> 4) & m, x1.x, p, false);
    p = __builtin_amdgcn_sdot4((int)((unsigned)w.y >> 4) & m, x1.y, p, false);
    p = __builtin_amdgcn_sdot4((int)((unsigned)w.z >> 4) & m, x1.z, p, false);
    p = __builtin_amdgcn_sdot4((int)((unsigned)w.w >> 4) & m, x1.w, p, false);
    return p;
}

// ---- int8 GEMV -----------------------------------------------------------------
//
// A workgroup of 256 lanes = 4 waves; each wave is 64/LPR groups of LPR lanes,
// a group owns R consecutive rows and its lanes take the blocks cyclically
// (lane l: blocks l, l+LPR, ...), so one wave-wide 128-bit load reads
// contiguous weight bytes. The row is walked in chunks of LPR*BPL blocks; a
// chunk's loads (BPL blocks per lane per row, plus the activation blocks)
// are all issued before any is used, so a lane waits on memory once per
// chunk rather than once per block. Per block and row: the int32 dot, then
// acc += (s_w * s_x) * P (+ bias * s_x * sum q_x) in f64. The group's lanes
// are summed in f64 with the DPP tree (group_sum_f64) and the sum is rounded
// once.
template <int DT, int M, int R, int LPR, int BPL>
__global__ __launch_bounds__(256) void gemv_i8_kernel(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ sc,
                                                      const uint16_t* __restrict__ bi, const int8_t* __restrict__ aq,
                                                      const double* __restrict__ asx, int rows, int nb,
                                                      float* __restrict__ y, size_t y_stride) {
    constexpr int G = 64 / LPR;
    constexpr int QV = DT == 1 ? 2 : 1;  // 16-byte loads per block of weights
    const int lane = threadIdx.x % LPR;
    const int grp = threadIdx.x / LPR;  // 0 .. 4*G-1
    const int row0 = (blockIdx.x * (4 * G) + grp) * R;
    const size_t cols = (size_t)nb * 32;
    const size_t qrow_bytes = DT == 1 ? cols : cols / 2;

    int rr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rr[r] = row0 + r < rows ? row0 + r : rows - 1;

    double acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0;

    for (int c0 = 0; c0 < nb; c0 += LPR * BPL) {
        int4 w[R][BPL][QV];
        uint32_t ws[R][BPL], wb[R][BPL];
        int4 x0[M][BPL], x1[M][BPL];
        double sxv[M][BPL], sxq[M][BPL];
        bool ok[BPL];
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int braw = c0 + lane + i * LPR;
            ok[i] = braw < nb;
            const size_t b = ok[i] ? braw : nb - 1;  // in bounds; skipped below
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const int4* xp = (const int4*)(aq + (size_t)m * cols + 32 * b);
                x0[m][i] = xp[0];
                x1[m][i] = xp[1];
                sxv[m][i] = asx[2 * ((size_t)m * nb + b)];
                sxq[m][i] = asx[2 * ((size_t)m * nb + b) + 1];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int4* wp = (const int4*)(qs + (size_t)rr[r] * qrow_bytes + (DT == 1 ? 32 : 16) * b);
#pragma unroll
                for (int v = 0; v < QV; ++v) w[r][i][v] = wp[v];
                ws[r][i] = sc[(size_t)rr[r] * nb + b];
                if (DT == 2) wb[r][i] = bi[(size_t)rr[r] * nb + b];
            }
        }
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            if (!ok[i]) continue;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const double sw = (double)bf16f(ws[r][i]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int P = DT == 1 ? dot_q8(w[r][i][0], w[r][i][QV - 1], x0[m][i], x1[m][i])
                                          : dot_q4(w[r][i][0], x0[m][i], x1[m][i]);
                    acc[r][m] = __builtin_fma(sw * sxv[m][i], (double)P, acc[r][m]);
                }
                if (DT == 2) {
                    const double bw = (double)bf16f(wb[r][i]);
#pragma unroll
                    for (int m = 0; m < M; ++m) acc[r][m] = __builtin_fma(bw, sxq[m][i], acc[r][m]);
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            double v = acc[r][m];
            // The DPP tree over the row's LPR lanes (at 64 lanes that of
            // every 64-lane int8 kernel, so their bits agree).
            v = group_sum_f64<LPR>(v);
            acc[r][m] = v;
        }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < rows)
#pragma unroll
                for (int m = 0; m < M; ++m) y[(size_t)m * y_stride + row0 + r] = (float)acc[r][m];
    }
}

// The same computation with three changes for short launches: the chunk
// loop has no tail (nb is a multiple of LPR*BPL, checked by the launcher),
// Q4 scale and bias come as one packed 32-bit word per block (`sb`,
// scale | bias << 16, built at upload), and the lane sum uses DPP. One
// vector in one chunk reads its activations from an LDS copy.
template <int DT, int M, int R, int LPR, int BPL, bool PF>
__global__ __launch_bounds__(256) void gemv_i8_v2_kernel(const uint8_t* __restrict__ qs,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint32_t* __restrict__ sb,
                                                         const int8_t* __restrict__ aq,
                                                         const double* __restrict__ asx, int rows, int nb,
                                                         float* __restrict__ y, size_t y_stride) {
    constexpr int G = 64 / LPR;
    constexpr int QV = DT == 1 ? 2 : 1;
    const int lane = threadIdx.x % LPR;
    const int grp = threadIdx.x / LPR;
    const int row0 = (blockIdx.x * (4 * G) + grp) * R;
    const size_t cols = (size_t)nb * 32;
    const size_t qrow_bytes = DT == 1 ? cols : cols / 2;

    int rr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rr[r] = row0 + r < rows ? row0 + r : rows - 1;

    double acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0;

    // One chunk's operands; with PF (rows of several chunks per lane) the
    // next chunk's loads are issued before the current chunk's arithmetic.
    struct Chunk {
        int4 w[R][BPL][QV];
        uint32_t s[R][BPL];
        int4 x0[M][BPL], x1[M][BPL];
        double2 sx[M][BPL];
    };
    auto load = [&](Chunk& k, int c0) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const size_t b = c0 + lane + i * LPR;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int4* wp = (const int4*)(qs + (size_t)rr[r] * qrow_bytes + (DT == 1 ? 32 : 16) * b);
#pragma unroll
                for (int v = 0; v < QV; ++v) k.w[r][i][v] = load_nt16(wp + v);
                k.s[r][i] = DT == 1 ? (uint32_t)sc[(size_t)rr[r] * nb + b] : sb[(size_t)rr[r] * nb + b];
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const int4* xp = (const int4*)(aq + (size_t)m * cols + 32 * b);
                k.x0[m][i] = xp[0];
                k.x1[m][i] = xp[1];
                k.sx[m][i] = ((const double2*)asx)[(size_t)m * nb + b];
            }
        }
    };
    auto run = [&](const Chunk& k) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const double sw = (double)bf16f(k.s[r][i] & 0xffffu);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int P = DT == 1 ? dot_q8(k.w[r][i][0], k.w[r][i][QV - 1], k.x0[m][i], k.x1[m][i])
                                          : dot_q4(k.w[r][i][0], k.x0[m][i], k.x1[m][i]);
                    acc[r][m] = __builtin_fma(sw * k.sx[m][i].x, (double)P, acc[r][m]);
                }
                if (DT == 2) {
                    const double bw = (double)bf16f(k.s[r][i] >> 16);
#pragma unroll
                    for (int m = 0; m < M; ++m) acc[r][m] = __builtin_fma(bw, k.sx[m][i].y, acc[r][m]);
                }
            }
        }
    };
    constexpr int STEP = LPR * BPL;
    if (PF) {
        // Every load in the loop is unconditional (the chunk after the pair
        // exists), so the compiler's waits count the chunk in flight behind
        // the one used: a load under a condition would make it wait for
        // everything. The last one or two chunks after the loop. (Two
        // chunks in flight, three buffers in turn, measured slower.)
        const int n = nb / STEP;  // whole chunks (nb is a multiple of STEP), at least 2
        Chunk A, B;
        load(A, 0);
        int c = 0;
        for (; c + 2 < n; c += 2) {
            load(B, (c + 1) * STEP);
            run(A);
            load(A, (c + 2) * STEP);
            run(B);
        }
        if (c + 1 < n) {
            load(B, (c + 1) * STEP);
            run(A);
            run(B);
        } else {
            run(A);
        }
    } else if constexpr (M == 1) {
        // One vector, one chunk (the launcher's shapes without PF): the
        // activations are copied to LDS once per workgroup (direct-to-LDS
        // loads, then the chunk's weight requests, then a wait for the
        // copies alone), so the lanes' activation reads stay off the
        // texture path that the weight stream uses.
        extern __shared__ __align__(16) unsigned char v2_smem[];
        const size_t xq_bytes = (cols + 1023) & ~(size_t)1023;
        {
            const int wave = threadIdx.x >> 6, ln = threadIdx.x & 63;
            for (size_t c = wave; c * 1024 < cols; c += 4) copy_1k(aq, cols, c * 1024, v2_smem + c * 1024, ln);
            for (size_t c = wave; c * 1024 < (size_t)nb * 16; c += 4)
                copy_1k(asx, (size_t)nb * 16, c * 1024, v2_smem + xq_bytes + c * 1024, ln);
        }
        int4 w[R][BPL][QV];
        uint32_t s[R][BPL];
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const size_t b = lane + i * LPR;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int4* wp = (const int4*)(qs + (size_t)rr[r] * qrow_bytes + (DT == 1 ? 32 : 16) * b);
#pragma unroll
                for (int v = 0; v < QV; ++v) w[r][i][v] = load_nt16(wp + v);
                s[r][i] = DT == 1 ? (uint32_t)sc[(size_t)rr[r] * nb + b] : sb[(size_t)rr[r] * nb + b];
            }
        }
        wait_vm_keep<R * BPL * (QV + 1)>(qs, DT == 1 ? (const void*)sc : (const void*)sb);
        __syncthreads();
        const int8_t* xq = (const int8_t*)v2_smem;
        const double2* xsx = (const double2*)(v2_smem + xq_bytes);
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const size_t b = lane + i * LPR;
            const int4 x0 = ((const int4*)(xq + 32 * b))[0], x1 = ((const int4*)(xq + 32 * b))[1];
            const double2 sx = xsx[b];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const double sw = (double)bf16f(s[r][i] & 0xffffu);
                const int P = DT == 1 ? dot_q8(w[r][i][0], w[r][i][QV - 1], x0, x1) : dot_q4(w[r][i][0], x0, x1);
                acc[r][0] = __builtin_fma(sw * sx.x, (double)P, acc[r][0]);
                if (DT == 2) acc[r][0] = __builtin_fma((double)bf16f(s[r][i] >> 16), sx.y, acc[r][0]);
            }
        }
    } else {
        for (int c0 = 0; c0 < nb; c0 += STEP) {
            int4 w[R][BPL][QV];
            uint32_t s[R][BPL];
            int4 x0[M][BPL], x1[M][BPL];
            double2 sx[M][BPL];
#pragma unroll
            for (int i = 0; i < BPL; ++i) {
                const size_t b = c0 + lane + i * LPR;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int4* wp = (const int4*)(qs + (size_t)rr[r] * qrow_bytes + (DT == 1 ? 32 : 16) * b);
#pragma unroll
                    for (int v = 0; v < QV; ++v) w[r][i][v] = load_nt16(wp + v);
                    s[r][i] = DT == 1 ? (uint32_t)sc[(size_t)rr[r] * nb + b] : sb[(size_t)rr[r] * nb + b];
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int4* xp = (const int4*)(aq + (size_t)m * cols + 32 * b);
                    x0[m][i] = xp[0];
                    x1[m][i] = xp[1];
                    sx[m][i] = ((const double2*)asx)[(size_t)m * nb + b];
                }
            }
#pragma unroll
            for (int i = 0; i < BPL; ++i) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const double sw = (double)bf16f(s[r][i] & 0xffffu);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const int P = DT == 1 ? dot_q8(w[r][i][0], w[r][i][QV - 1], x0[m][i], x1[m][i])
                                              : dot_q4(w[r][i][0], x0[m][i], x1[m][i]);
                        acc[r][m] = __builtin_fma(sw * sx[m][i].x, (double)P, acc[r][m]);
                    }
                    if (DT == 2) {
                        const double bw = (double)bf16f(s[r][i] >> 16);
#pragma unroll
                        for (int m = 0; m < M; ++m) acc[r][m] = __builtin_fma(bw, sx[m][i].y, acc[r][m]);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = group_sum_f64<LPR>(acc[r][m]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < rows)
#pragma unroll
                for (int m = 0; m < M; ++m) y[(size_t)m * y_stride + row0 + r] = (float)acc[r][m];
    }
}

// P[t][r][b], one thread per (t, r, b), with the path's dot routines.
template <int DT>
__global__ void block_dots_kernel(const uint8_t* __restrict__ qs, const int8_t* __restrict__ aq, int rows, int nb,
                                  int n_tok, int32_t* __restrict__ P) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t per = (size_t)rows * nb;
    if (idx >= per * n_tok) return;
    size_t t = idx / per, rb = idx - t * per;
    size_t r = rb / nb, b = rb - r * nb;
    const size_t cols = (size_t)nb * 32;
    const int4* xp = (const int4*)(aq + t * cols + 32 * b);
    int4 x0 = xp[0], x1 = xp[1];
    if (DT == 1) {
        const int4* wp = (const int4*)(qs + r * cols + 32 * b);
        P[idx] = dot_q8(wp[0], wp[1], x0, x1);
    } else {
        P[idx] = dot_q4(*(const int4*)(qs + r * cols / 2 + 16 * b), x0, x1);
    }
}

template <int DT, int M, int R, int LPR, int BPL>
void launch_cfg(const uint8_t* qs, const uint16_t* sc, const uint16_t* bi, const int8_t* aq, const double* asx,
                int rows, int nb, float* y, size_t ys, hipStream_t st) {
    constexpr int rows_per_wg = 4 * (64 / LPR) * R;
    gemv_i8_kernel<DT, M, R, LPR, BPL>
        <<<ceil_div(rows, rows_per_wg), 256, 0, st>>>(qs, sc, bi, aq, asx, rows, nb, y, ys);
}

// Launch shape by row length: lanes per row and blocks per lane so that a
// lane's whole row share is one chunk of hoisted loads, with blocks per lane
// = ceil(nb / lanes) so no lane issues a load past the row (measured on the
// 262144 x 1152 Q8 vocab GEMV, nb = 36: 3 blocks per lane 51.8 us against
// 4 blocks 58.6 us). A lane's blocks and their order do not depend on the
// chunking, so neither do the results. One vector with 97..127 blocks
// (Qwen2.5-7B's 3584 columns) or Q8 rows past 256 blocks (its 18944-column
// down projection): the best of 8 shapes measured at those matrices, Q8
// 3584x3584 / 4608x3584 / 37888x3584 / 3584x18944 5.28 / 6.87 / 24.9 / 16.5
// -> 4.86 / 5.38 / 23.7 / 15.6 us, Q4 3584x3584 / 37888x3584 4.36 / 16.4 ->
// 4.17 / 16.2 us.
template <int DT, int M>
void launch_m(const uint8_t* qs, const uint16_t* sc, const uint16_t* bi, const int8_t* aq, const double* asx,
              int rows, int nb, float* y, size_t ys, hipStream_t st) {
    if constexpr (M == 1) {
        if (nb > 96 && nb <= 128) {
            if (DT == 1)
                launch_cfg<DT, M, 1, 64, 2>(qs, sc, bi, aq, asx, rows, nb, y, ys, st);
            else
                launch_cfg<DT, M, 2, 64, 2>(qs, sc, bi, aq, asx, rows, nb, y, ys, st);
            return;
        }
        if (DT == 1 && nb > 256) {
            launch_cfg<DT, M, 2, 64, 5>(qs, sc, bi, aq, asx, rows, nb, y, ys, st);
            return;
        }
    }
    if (nb <= 64) {
        switch (ceil_div(nb, 16)) {
        case 1: launch_cfg<DT, M, 2, 16, 1>(qs, sc, bi, aq, asx, rows, nb, y, ys, st); break;
        case 2: launch_cfg<DT, M, 2, 16, 2>(qs, sc, bi, aq, asx, rows, nb, y, ys, st); break;
        case 3: launch_cfg<DT, M, 2, 16, 3>(qs, sc, bi, aq, asx, rows, nb, y, ys, st); break;
        default: launch_cfg<DT, M, 2, 16, 4>(qs, sc, bi, aq, asx, rows, nb, y, ys, st); break;
        }
    } else if (nb <= 128) {
        if (nb <= 96)
            launch_cfg<DT, M, 2, 32, 3>(qs, sc, bi, aq, asx, rows, nb, y, ys, st);
        else
            launch_cfg<DT, M, 2, 32, 4>(qs, sc, bi, aq, asx, rows, nb, y, ys, st);
    } else {
        launch_cfg<DT, M, 2, 64, 4>(qs, sc, bi, aq, asx, rows, nb, y, ys, st);
    }
}

// sb[i] = scale[i] | bias[i] << 16: one 32-bit load per Q4 block.
__global__ void pack_sb_kernel(const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
                               uint32_t* __restrict__ sb, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) sb[i] = (uint32_t)sc[i] | ((uint32_t)bi[i] << 16);
}

template <int DT, int M, int R, int LPR, int BPL>
void launch_v2(const uint8_t* qs, const uint16_t* sc, const uint32_t* sb, const int8_t* aq, const double* asx,
               int rows, int nb, float* y, size_t ys, hipStream_t st) {
    constexpr int rows_per_wg = 4 * (64 / LPR) * R;
    if (nb > LPR * BPL) {
        gemv_i8_v2_kernel<DT, M, R, LPR, BPL, true>
            <<<ceil_div(rows, rows_per_wg), 256, 0, st>>>(qs, sc, sb, aq, asx, rows, nb, y, ys);
    } else {
        // One vector: the activation copy in LDS (quants, then the pairs).
        const size_t lds = M == 1 ? (((size_t)nb * 32 + 1023) & ~(size_t)1023) + (((size_t)nb * 16 + 1023) & ~(size_t)1023)
                                  : 0;
        gemv_i8_v2_kernel<DT, M, R, LPR, BPL, false>
            <<<ceil_div(rows, rows_per_wg), 256, lds, st>>>(qs, sc, sb, aq, asx, rows, nb, y, ys);
    }
}

// Launch shape from the measured sweep (Llama-3-8B and vocab shapes): 64
// lanes per row taking 2 blocks per chunk when the row is a whole number of
// 128-block chunks, else 1; two rows per lane group for tall matrices.
template <int DT, int M>
bool launch_v2_m(const uint8_t* qs, const uint16_t* sc, const uint32_t* sb, const int8_t* aq, const double* asx,
                 int rows, int nb, float* y, size_t ys, hipStream_t st) {
    if (nb % 64 != 0) return false;
    const bool tall = rows >= 8192;
    if (nb % 128 == 0) {
        if (tall) launch_v2<DT, M, 2, 64, 2>(qs, sc, sb, aq, asx, rows, nb, y, ys, st);
        else launch_v2<DT, M, 1, 64, 2>(qs, sc, sb, aq, asx, rows, nb, y, ys, st);
    } else {
        if (tall) launch_v2<DT, M, 2, 64, 1>(qs, sc, sb, aq, asx, rows, nb, y, ys, st);
        else launch_v2<DT, M, 2, 64, 1>(qs, sc, sb, aq, asx, rows, nb, y, ys, st);
    }
    return true;
}


// ---- int8 GEMV with the residual add, RMSNorm and quantizer fused -----------
//
// One vector, rows of 97 .. 256 blocks, where the plain GEMV runs 64 lanes
// per row (lane l summing blocks l, l + 64, ... in that order) and reduces
// the lanes with the DPP tree (group_sum_f64): the same per-lane order and
// tree here, so the results are the bits of the device forward's norm,
// the quantizer and the plain GEMV run one after another. One workgroup of
// 16 waves per CU forms the int8 input: its threads load their pieces of x,
// r and gamma, then each wave requests its first weights, which are in
// flight while wave 0 runs the sum of squares (the device forward's order,
// rmsnorm_exact.h, from a chain-major copy in LDS) and the normed row is
// quantized into LDS with the library quantizer's encoder (q8_act.h). Each
// wave then takes row groups of R rows grid-stride, the next chunk's
// weights in flight while the current one is summed.
constexpr int I8N_T = 1024;  // threads per workgroup
template <int DT, int R, int BPL, int K4>
__global__ __launch_bounds__(I8N_T) void gemv_i8_norm_kernel(const uint8_t* __restrict__ qs,
                                                             const uint16_t* __restrict__ sc,
                                                             const uint32_t* __restrict__ sb, int rows, int nb,
                                                             float* __restrict__ y, NormIn nrm) {
    constexpr int QV = DT == 1 ? 2 : 1;
    constexpr int STEP = 64 * BPL;
    constexpr int NW = I8N_T / 64;
    extern __shared__ __align__(16) unsigned char i8n_smem[];
    __shared__ float nsc;
    const int tid = threadIdx.x, lane = tid & 63;
    const int cols = nb * 32, n4 = cols / 4, ts = rms_t_stride(cols);
    const size_t qrow_bytes = DT == 1 ? (size_t)cols : (size_t)cols / 2;
    float* xt = (float*)i8n_smem;                                  // x (+ r), chain-major: [8][ts]
    int8_t* xq = (int8_t*)(i8n_smem + (size_t)32 * ts);            // the quants
    double2* xsx = (double2*)(i8n_smem + (size_t)32 * ts + cols);  // per block: scale, scale * sum of quants

    // Piece k of this thread: values 4i .. 4i + 3, i = tid + I8N_T k.
    float4 xv[K4], rv[K4], gv[K4];
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int i = tid + I8N_T * k;
        if (i < n4) {
            xv[k] = ((const float4*)nrm.x)[i];
            gv[k] = ((const float4*)nrm.gamma)[i];
            if (nrm.r) rv[k] = ((const float4*)nrm.r)[i];
        }
    }
    // Every wave's piece loads are issued before any weight load (an
    // execution barrier only: nothing waits for the loads here), so waiting
    // for the pieces waits neither for this wave's weights (loads complete
    // in issue order) nor behind other waves' in the CU's memory pipeline.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    struct Chunk {
        int4 w[R][BPL][QV];
        uint32_t s[R][BPL];
    };
    const int ng = (rows + R - 1) / R, gstep = gridDim.x * NW;
    auto load = [&](Chunk& k, int g, int c0) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int braw = c0 + lane + 64 * i;
            const size_t b = braw < nb ? braw : nb - 1;  // in bounds; skipped by run
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const size_t rw = g * R + r < rows ? g * R + r : rows - 1;
                const int4* wp = (const int4*)(qs + rw * qrow_bytes + (DT == 1 ? 32 : 16) * b);
#pragma unroll
                for (int v = 0; v < QV; ++v) k.w[r][i][v] = load_nt16(wp + v);
                k.s[r][i] = DT == 1 ? (uint32_t)sc[rw * nb + b] : sb[rw * nb + b];
            }
        }
    };
    double acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0;
    // The block terms in gemv_i8_kernel's order: per block, per row, the
    // scaled dot, then (Q4) the bias term.
    auto run = [&](const Chunk& k, int c0) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int b = c0 + lane + 64 * i;
            if (b >= nb) continue;
            const int4 x0 = ((const int4*)(xq + 32 * b))[0], x1 = ((const int4*)(xq + 32 * b))[1];
            const double2 sx = xsx[b];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const double sw = (double)bf16f(k.s[r][i] & 0xffffu);
                const int P = DT == 1 ? dot_q8(k.w[r][i][0], k.w[r][i][QV - 1], x0, x1)
                                      : dot_q4(k.w[r][i][0], x0, x1);
                acc[r] = __builtin_fma(sw * sx.x, (double)P, acc[r]);
                if (DT == 2) acc[r] = __builtin_fma((double)bf16f(k.s[r][i] >> 16), sx.y, acc[r]);
            }
        }
    };
    auto finish = [&](int g) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            double v = acc[r];
            v = group_sum_f64<64>(v);
            if (lane == 0 && g * R + r < rows) y[g * R + r] = (float)v;
            acc[r] = 0.0;
        }
    };

    const int g0 = blockIdx.x * NW + (tid >> 6);
    Chunk A, B;
    // Unconditional (a wave past the last row group rereads it, unused), so
    // the waits for the pieces below count these loads exactly.
    load(A, g0 < ng ? g0 : ng - 1, 0);

    // x + r into LDS chain-major (element e at (e mod 8) * ts + e / 8;
    // workgroup 0 also writes it out), the sum of squares, then the normed
    // pieces quantized into LDS.
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        const int i = tid + I8N_T * k;
        if (i < n4) {
            if (nrm.r)
                xv[k] = float4{__fadd_rn(xv[k].x, rv[k].x), __fadd_rn(xv[k].y, rv[k].y),
                               __fadd_rn(xv[k].z, rv[k].z), __fadd_rn(xv[k].w, rv[k].w)};
            float* d = xt + (size_t)(4 * (i & 1)) * ts + (i >> 1);
            d[0] = xv[k].x;
            d[ts] = xv[k].y;
            d[2 * ts] = xv[k].z;
            d[3 * ts] = xv[k].w;
            if (blockIdx.x == 0) {
                if (nrm.x_out) ((float4*)nrm.x_out)[i] = xv[k];
                if (nrm.rec) ((float4*)nrm.rec)[i] = xv[k];
            }
        }
    }
    __syncthreads();
    if (tid < 64) {
        // Shorter read batches where the chunk's registers are larger.
        const double ss = rms_sumsq_t<BPL == 2 ? 8 : 4>(xt, cols, tid);
        if (tid == 0) nsc = rms_scale(ss, cols, nrm.eps);
    }
    __syncthreads();
    const float scl = nsc;
    float4 o[K4];
#pragma unroll
    for (int k = 0; k < K4; ++k) {
        o[k] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (tid + I8N_T * k < n4)
            o[k] = float4{__fmul_rn(__fmul_rn(xv[k].x, scl), gv[k].x), __fmul_rn(__fmul_rn(xv[k].y, scl), gv[k].y),
                          __fmul_rn(__fmul_rn(xv[k].z, scl), gv[k].z), __fmul_rn(__fmul_rn(xv[k].w, scl), gv[k].w)};
    }
    q8_pieces<K4>(o, tid, I8N_T, n4, [&](int i, uint32_t word, const Q8Scale& s, int qsum) {
        ((uint32_t*)xq)[i] = word;
        if ((i & 7) == 0) xsx[i >> 3] = double2{(double)s.scale, (double)s.scale * (double)qsum};
    });
    __syncthreads();

    if (g0 >= ng) return;
    // Items (row group, chunk) in order; A holds the current item's
    // weights, B the next one's, then the roles swap. (Unconditional loads,
    // so that the compiler's waits count the item in flight, measured
    // slower here at the decode's shapes but one.)
    int ga = g0, ca = 0;
    while (true) {
        int gb = ga, cb = ca + STEP;
        if (cb >= nb) {
            cb = 0;
            gb += gstep;
        }
        const bool hb = gb < ng;
        if (hb) load(B, gb, cb);
        run(A, ca);
        if (ca + STEP >= nb) finish(ga);
        if (!hb) break;
        int gc = gb, cc = cb + STEP;
        if (cc >= nb) {
            cc = 0;
            gc += gstep;
        }
        const bool hc = gc < ng;
        if (hc) load(A, gc, cc);
        run(B, cb);
        if (cb + STEP >= nb) finish(gb);
        if (!hc) break;
        ga = gc;
        ca = cc;
    }
}

template <int DT, int R, int BPL, int K4>
void launch_i8n(const uint8_t* qs, const uint16_t* sc, const uint32_t* sb, const NormIn& nrm, int rows, int nb,
                float* y, hipStream_t st) {
    constexpr int NW = I8N_T / 64;
    const int want = ceil_div(ceil_div(rows, R), NW), cap = cu_count();
    const int grid = want < cap ? want : cap;
    const size_t lds = (size_t)32 * rms_t_stride(nb * 32) + (size_t)nb * 32 + (size_t)nb * 16;
    gemv_i8_norm_kernel<DT, R, BPL, K4><<<grid, I8N_T, lds, st>>>(qs, sc, sb, rows, nb, y, nrm);
}

// A row is one chunk: 128 blocks (up to 128-block rows, one piece per
// thread) or 256 blocks (two pieces, one row per group).
template <int DT>
void launch_i8n_dt(const uint8_t* qs, const uint16_t* sc, const uint32_t* sb, const NormIn& nrm, int rows, int nb,
                   float* y, hipStream_t st) {
    if (nb <= 128)
        launch_i8n<DT, DT == 1 ? 1 : 2, 2, 1>(qs, sc, sb, nrm, rows, nb, y, st);
    else
        launch_i8n<DT, 1, 4, 2>(qs, sc, sb, nrm, rows, nb, y, st);
}


// ---- int8 GEMV, one vector, activations staged in LDS, grid-stride rows -----
//
// Rows of 64-lane groups where the plain launch shapes below are weakest:
// Q8 rows of whole 64-block groups in tall matrices (8192+ rows) or of 256+
// blocks, Q4 rows of 257+ blocks that are not whole groups (3584+ rows).
// Measured against the plain path on one box, alternating (medians of 5):
// Q8 14336x4096 18.0 -> 13.5 us, 4096x14336 13.7 -> 12.7, Q4 3584x18944
// 11.9 -> 9.5; at Q8 4096-6144 rows of 128-192 blocks and Q8 3584x18944
// the two were within 0.6 us either way, so those stay plain. Up to two
// workgroups of 16 waves per CU (below 16 rows per CU, one per CU of
// ceil(rows / CUs) waves: i8_lds_waves); each copies the quantized activations
// (the quants and the (scale, scale * sum) pairs) into LDS once, then each
// wave takes rows grid-stride, chunks of 128 blocks with the next chunk's
// weights in flight. A lane sums blocks l, l + 64, ... in order and the
// lanes are reduced with the plain path's DPP tree, so the bits are the
// plain path's.
//
// K4 > 0: the vector arrives as f32 (xf) and the workgroup quantizes it
// itself with the library quantizer's encoder (q8_act.h), no separate
// quantizer launch: each thread loads its K4 pieces (values 4i .. 4i + 3,
// i = tid + T k for T threads; K4 * T >= nb * 8) before any weight load,
// and encodes them into LDS while its first weights are in flight.
constexpr int I8L_T = 1024;
template <int DT, int K4 = 0>
__global__ __launch_bounds__(I8L_T) void gemv_i8_lds_kernel(const uint8_t* __restrict__ qs,
                                                            const uint16_t* __restrict__ sc,
                                                            const uint32_t* __restrict__ sb,
                                                            const int8_t* __restrict__ aq,
                                                            const double* __restrict__ asx, int rows, int nb,
                                                            float* __restrict__ y, const float* __restrict__ xf) {
    constexpr int QV = DT == 1 ? 2 : 1;
    constexpr int BPL = 2, STEP = 64 * BPL;
    constexpr bool QX = K4 > 0;
    const int nt = blockDim.x, NW = nt >> 6;  // up to I8L_T threads
    extern __shared__ __align__(16) unsigned char i8l_smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t cols = (size_t)nb * 32, qrow_bytes = DT == 1 ? cols : cols / 2;
    int8_t* xq = (int8_t*)i8l_smem;
    double2* xsx = (double2*)(i8l_smem + ((cols + 1023) & ~(size_t)1023));
    const int n4 = nb * 8;
    float4 xv[QX ? K4 : 1];
    if constexpr (QX) {
        // Unconditional (indices clamped; pieces past n4 are not encoded),
        // and every wave's issued before any weight load (an execution
        // barrier only), so waiting for them waits for no weights.
#pragma unroll
        for (int k = 0; k < K4; ++k) {
            const int i = tid + nt * k;
            xv[k] = ((const float4*)xf)[i < n4 ? i : n4 - 1];
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    } else {
        for (size_t c = wave; c * 1024 < cols; c += NW)
            copy_1k(aq, cols, c * 1024, (unsigned char*)xq + c * 1024, lane);
        for (size_t c = wave; c * 1024 < (size_t)nb * 16; c += NW)
            copy_1k(asx, (size_t)nb * 16, c * 1024, (unsigned char*)xsx + c * 1024, lane);
    }

    struct Chunk {
        int4 w[BPL][QV];
        uint32_t s[BPL];
    };
    const int gstep = gridDim.x * NW;
    auto load = [&](Chunk& k, int row, int c0) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int braw = c0 + lane + 64 * i;
            const size_t b = braw < nb ? braw : nb - 1;  // in bounds; skipped by run
            const int4* wp = (const int4*)(qs + (size_t)row * qrow_bytes + (DT == 1 ? 32 : 16) * b);
#pragma unroll
            for (int v = 0; v < QV; ++v) k.w[i][v] = load_nt16(wp + v);
            k.s[i] = DT == 1 ? (uint32_t)sc[(size_t)row * nb + b] : sb[(size_t)row * nb + b];
        }
    };
    double acc = 0.0;
    // gemv_i8_kernel's block term order: the scaled dot, then (Q4) the bias term.
    auto run = [&](const Chunk& k, int c0) {
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int b = c0 + lane + 64 * i;
            if (b >= nb) continue;
            const int4 x0 = ((const int4*)(xq + 32 * b))[0], x1 = ((const int4*)(xq + 32 * b))[1];
            const double2 sx = xsx[b];
            const double sw = (double)bf16f(k.s[i] & 0xffffu);
            const int P = DT == 1 ? dot_q8(k.w[i][0], k.w[i][QV - 1], x0, x1) : dot_q4(k.w[i][0], x0, x1);
            acc = __builtin_fma(sw * sx.x, (double)P, acc);
            if (DT == 2) acc = __builtin_fma((double)bf16f(k.s[i] >> 16), sx.y, acc);
        }
    };
    auto finish = [&](int row) {
        double v = acc;
        v = group_sum_f64<64>(v);
        if (lane == 0) y[row] = (float)v;
        acc = 0.0;
    };

    const int r0 = blockIdx.x * NW + wave;
    Chunk A, B;
    // Unconditional (a wave past the last row rereads it, unused), so the
    // wait below counts these loads exactly; the copies land first.
    load(A, r0 < rows ? r0 : rows - 1, 0);
    if constexpr (QX) {
        q8_pieces<K4>(xv, tid, nt, n4, [&](int i, uint32_t word, const Q8Scale& s, int qsum) {
            ((uint32_t*)xq)[i] = word;
            if ((i & 7) == 0) xsx[i >> 3] = double2{(double)s.scale, (double)s.scale * (double)qsum};
        });
    } else {
        wait_vm_keep<BPL * (QV + 1)>(qs, DT == 1 ? (const void*)sc : (const void*)sb);
    }
    __syncthreads();
    if (r0 >= rows) return;
    // Items (row, chunk) in order; A holds the current item's weights, B
    // the next one's, then the roles swap. Q4: the loads are unconditional
    // (past the wave's last item a reread of the current one, unused), so
    // the compiler's waits count the item in flight (a load under a
    // condition makes each item wait for everything): Q4 3584x18944 10.5
    // -> 10.2 us, 3584x9216 6.65 -> 6.3. Q8 keeps the conditional loads:
    // with its chunks (twice Q4's bytes) in flight as well, 14336x4096 went
    // 14.7 -> 18.8 us and 3584x10240 10.0 -> 10.55.
    constexpr bool EXACT = DT == 2;
    int ra = r0, ca = 0;
    while (true) {
        int rb = ra, cb = ca + STEP;
        if (cb >= nb) {
            cb = 0;
            rb += gstep;
        }
        const bool hb = rb < rows;
        if (EXACT)
            load(B, hb ? rb : ra, hb ? cb : ca);
        else if (hb)
            load(B, rb, cb);
        run(A, ca);
        if (ca + STEP >= nb) finish(ra);
        if (!hb) break;
        int rc = rb, cc = cb + STEP;
        if (cc >= nb) {
            cc = 0;
            rc += gstep;
        }
        const bool hc = rc < rows;
        if (EXACT)
            load(A, hc ? rc : rb, hc ? cc : cb);
        else if (hc)
            load(A, rc, cc);
        run(B, cb);
        if (cb + STEP >= nb) finish(rb);
        if (!hc) break;
        ra = rc;
        ca = cc;
    }
}

constexpr int I8L_WG_PER_CU = 2;

// The shapes where the staged kernel measured faster (the plain path runs
// 64 lanes per row at all of them, so the lane order is the same).
bool i8_lds_shape(int dtype, int rows, int nb) {
    if (dtype == 1) return nb % 64 == 0 && nb >= 128 && (rows >= 8192 || (nb >= 256 && rows >= 3584));
    return nb > 256 && nb % 64 != 0 && rows >= 3584;
}

// Workgroups resident per CU (at most I8L_WG_PER_CU), from the instance's
// registers and LDS: the grid is never larger than what runs at once.
template <int DT, int K4>
int i8_lds_per_cu(size_t lds) {
    static int n = -1;
    if (n < 0) {
        int b = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, gemv_i8_lds_kernel<DT, K4>, I8L_T, lds) !=
                hipSuccess ||
            b < 1)
            b = 1;
        n = b < I8L_WG_PER_CU ? b : I8L_WG_PER_CU;
    }
    return n;
}

// Waves per workgroup: 16, except that below 16 rows per CU the rows are
// spread over every CU (ceil(rows / CUs) waves, at least 8), so that no CU
// sits idle while others take two rows per wave (3584 rows: 256 workgroups
// of 14 waves, not 224 of 16).
inline int i8_lds_waves(int rows) {
    const int cus = cu_count();
    if (rows >= 16 * cus) return 16;
    const int w = ceil_div(rows, cus);
    return w < 8 ? 8 : w;
}

template <int DT, int K4 = 0>
void launch_i8_lds(const uint8_t* qs, const uint16_t* sc, const uint32_t* sb, const int8_t* aq, const double* asx,
                   int rows, int nb, float* y, hipStream_t st, const float* xf = nullptr) {
    const size_t lds = (((size_t)nb * 32 + 1023) & ~(size_t)1023) + (((size_t)nb * 16 + 1023) & ~(size_t)1023);
    const int waves = i8_lds_waves(rows);
    const int want = ceil_div(rows, waves), cap = i8_lds_per_cu<DT, K4>(lds) * cu_count();
    const int grid = want < cap ? want : cap;
    gemv_i8_lds_kernel<DT, K4><<<grid, 64 * waves, lds, st>>>(qs, sc, sb, aq, asx, rows, nb, y, xf);
}

// The quantizing prologue's pieces per thread: K4 * threads >= nb * 8.
template <int DT>
void launch_i8_qx_k(const uint8_t* qs, const uint16_t* sc, const uint32_t* sb, const float* x, int rows, int nb,
                    float* y, hipStream_t st) {
    const int need = ceil_div(nb * 8, 64 * i8_lds_waves(rows));
    if (need <= 1) launch_i8_lds<DT, 1>(qs, sc, sb, nullptr, nullptr, rows, nb, y, st, x);
    else if (need <= 2) launch_i8_lds<DT, 2>(qs, sc, sb, nullptr, nullptr, rows, nb, y, st, x);
    else if (need <= 3) launch_i8_lds<DT, 3>(qs, sc, sb, nullptr, nullptr, rows, nb, y, st, x);
    else if (need <= 4) launch_i8_lds<DT, 4>(qs, sc, sb, nullptr, nullptr, rows, nb, y, st, x);
    else launch_i8_lds<DT, 6>(qs, sc, sb, nullptr, nullptr, rows, nb, y, st, x);
}
}  // namespace

// One vector, rows of 97+ blocks (the plain path's 64 lanes per row, so its
// lane order and tree). Every workgroup encodes the whole vector, so the
// encoding's VALU work per CU grows with the row: against the quantizer
// launch followed by the GEMV (bench.py --workload i8_prologue: HIP graphs
// of launches on rotating weights) the prologue is faster up to 288 blocks
// (Q4 4608x3584 7.37 -> 5.13 us, 3584x3584 6.69 -> 3.76, 4096x8192 8.56 ->
// 6.77, 3584x9216 8.85 -> 8.05; Q8 4608x3584 7.78 -> 7.02, 14336x4096
// 15.80 -> 13.38, 3584x9216 11.46 -> 10.73); rows of 448 and 592 blocks
// (14336 and 18944 columns) and tall Q8 matrices of rows that are not whole
// 64-block groups (Q8 37888x3584) measured slower with it, so they keep the
// two launches.
bool launch_gemv_i8_qx(int dtype, const uint8_t* qs, const uint16_t* scales, const uint32_t* sb, const float* x,
                       int rows, int nb, float* y, hipStream_t st) {
    if (nb <= 96 || nb > 384 || (dtype == 2 && !sb) || ((uintptr_t)x & 15) != 0) return false;
    if (dtype == 1 && rows >= 16384 && nb % 64 != 0) return false;
    if (dtype == 1)
        launch_i8_qx_k<1>(qs, scales, sb, x, rows, nb, y, st);
    else
        launch_i8_qx_k<2>(qs, scales, sb, x, rows, nb, y, st);
    return true;
}

void launch_pack_sb(const uint16_t* sc, const uint16_t* bi, uint32_t* sb, size_t n, hipStream_t st) {
    pack_sb_kernel<<<(int)((n + 255) / 256), 256, 0, st>>>(sc, bi, sb, n);
}

void launch_quantize_act(const float* x, size_t x_stride, int cols, int n_tok, int8_t* q, uint16_t* s, double* sx,
                         float* sxT, int tok_pad, hipStream_t st) {
    int blocks = (cols / 32) * n_tok;
    quantize_act_kernel<<<ceil_div(blocks, 8), 256, 0, st>>>(x, x_stride, cols, n_tok, q, s, sx, sxT, tok_pad);
}

void launch_gemv_i8(int dtype, const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const uint32_t* sb,
                    const int8_t* aq, const double* asx, int rows, int nb, int n_tok, float* y, size_t y_stride,
                    hipStream_t st) {
    // One vector at the staged kernel's shapes (x and its pairs in LDS: up
    // to 32768 columns).
    if (n_tok == 1 && i8_lds_shape(dtype, rows, nb) && nb * 32 <= 32768 && (dtype == 1 || sb)) {
        if (dtype == 1)
            launch_i8_lds<1>(qs, scales, sb, aq, asx, rows, nb, y, st);
        else
            launch_i8_lds<2>(qs, scales, sb, aq, asx, rows, nb, y, st);
        return;
    }
    const size_t cols = (size_t)nb * 32;
    for (int t0 = 0; t0 < n_tok; t0 += 4) {
        int m = n_tok - t0 < 4 ? n_tok - t0 : 4;
        const int8_t* a = aq + (size_t)t0 * cols;
        const double* s = asx + 2 * (size_t)t0 * nb;
        float* yt = y + (size_t)t0 * y_stride;
#define NNH_L(DT, M)                                                                             \
    do {                                                                                         \
        if (!launch_v2_m<DT, M>(qs, scales, sb, a, s, rows, nb, yt, y_stride, st))                \
            launch_m<DT, M>(qs, scales, biases, a, s, rows, nb, yt, y_stride, st);               \
    } while (0)
        if (dtype == 1) {
            if (m == 1) NNH_L(1, 1); else if (m == 2) NNH_L(1, 2); else if (m == 3) NNH_L(1, 3); else NNH_L(1, 4);
        } else {
            if (m == 1) NNH_L(2, 1); else if (m == 2) NNH_L(2, 2); else if (m == 3) NNH_L(2, 3); else NNH_L(2, 4);
        }
#undef NNH_L
    }
}

bool launch_gemv_i8_norm(int dtype, const uint8_t* qs, const uint16_t* scales, const uint32_t* sb,
                         const NormIn& nrm, int rows, int nb, float* y, hipStream_t st) {
    const auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (nb <= 96 || nb > 256 || (dtype == 2 && !sb)) return false;
    if (!aligned(nrm.x) || !aligned(nrm.gamma) || !aligned(nrm.r) || !aligned(nrm.x_out) || !aligned(nrm.rec))
        return false;
    if (dtype == 1)
        launch_i8n_dt<1>(qs, scales, sb, nrm, rows, nb, y, st);
    else
        launch_i8n_dt<2>(qs, scales, sb, nrm, rows, nb, y, st);
    return true;
}

void launch_block_dots(int dtype, const uint8_t* qs, const int8_t* aq, int rows, int nb, int n_tok, int32_t* P,
                       hipStream_t st) {
    size_t n = (size_t)rows * nb * n_tok;
    int blocks = (int)((n + 255) / 256);
    if (dtype == 1)
        block_dots_kernel<1><<<blocks, 256, 0, st>>>(qs, aq, rows, nb, n_tok, P);
    else
        block_dots_kernel<2><<<blocks, 256, 0, st>>>(qs, aq, rows, nb, n_tok, P);
}

}  // namespace nnh
