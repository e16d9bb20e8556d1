// The int8 MFMA GEMM for many activation vectors (prefill, batched verify):
// y[m][n] = sum_b s_x[m,b] s_w[n,b] P_b[m][n]  (+ Q4: sum_b bias[n,b] s_x[m,b] sum_k q_x[m,32b+k]),
// P_b[m][n] = sum_k q_w[n,32b+k] q_x[m,32b+k], exact in int32.
//
// One v_mfma_i32_32x32x32_i8 is one nncpu block (K = 32) of a 32 x 32 tile,
// so its result is exactly the tile's block dots P_b. The A operand is the
// weights (rows n), B the activations (tokens m); lane l holds row / token
// l%32 and K-half l/32 (16 bytes). Result element (i, j) sits in lane
// j + 32h, register r, with i = (r/4)*8 + 4h + r%4: a lane owns one token
// and 16 weight rows of each 32 x 32 tile.
//
// Epilogue per block and output: acc = fma(P, s_w * s_x, acc) (+ Q4
// acc = fma(bias, s_x * sum q_x, acc)) in f64; P and the scale products are
// exact, so every output is within one f32 ulp of the exact sum (an f32 sum
// over K = 18944 would take most of the 1e-5 tolerance next to nncpu's own
// f32 rounding). nncpu's per-32 BF16 scales make this epilogue, not the
// MFMA, the compute bound: 4 (Q8) / 5 (Q4) VALU ops per output and block
// against 32 MACs.
//
// Workgroup: 128 weight rows x 128 tokens, 4 waves as 2 x 2, each wave a
// 64 x 64 block of 2 x 2 MFMA tiles. The K loop runs over chunks of KB
// blocks through a ring of three LDS stages filled by direct global -> LDS
// loads (global_load_lds_dwordx4, no staging registers), so two chunks are
// in flight while one is computed. Scales come from block-major f32 copies
// (weights: built at upload; activations: written by the quantizer) so each
// stage's scales are contiguous 16-byte pieces too.

#include "common.h"

namespace nnh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int TILE = 128;  // weight rows and tokens per workgroup

template <int DT, int KB>
struct GStage {
    static constexpr int QB = DT == 1 ? 32 : 16;  // weight bytes per row and block
    uint8_t A[KB * TILE * QB];                    // [blk][row][QB]
    int8_t B[KB * TILE * 32];                     // [blk][token][32]
    float SW[KB * TILE];                          // [blk][row]
    float SX[KB * TILE];                          // [blk][token]
    float BI[DT == 2 ? KB * TILE : 4];            // [blk][row]   (Q4)
    float SXQ[DT == 2 ? KB * TILE : 4];           // [blk][token] (Q4)
};

// Direct-load instructions per stage (64 lanes x 16 bytes each).
template <int DT, int KB>
struct GPlan {
    static constexpr int I_A = KB * TILE * GStage<DT, KB>::QB / 16 / 64;
    static constexpr int I_B = KB * TILE * 32 / 16 / 64;
    static constexpr int I_S = KB * TILE * 4 / 16 / 64;  // one f32 [blk][TILE] table
    static constexpr int I_TOTAL = I_A + I_B + (DT == 2 ? 4 : 2) * I_S;
    static constexpr int PER_WAVE = I_TOTAL / 4;
    static_assert(I_A % 4 == 0 && I_B % 4 == 0 && I_TOTAL % 4 == 0, "stage loads must split evenly over 4 waves");
    static_assert(I_S >= 1 && KB * TILE * 4 % 1024 == 0, "scale tables must fill whole load instructions");
    static_assert(2 * PER_WAVE < 64, "vmcnt holds at most 63");
};

struct GArgs {
    const uint8_t* qs;  // weights, nncpu row-major quants
    const float* swT;   // [nb][rows_pad] weight scales; Q4 biases follow at + nb * rows_pad
    const int8_t* aq;   // activation quants [n_tok][cols]
    const float* sxT;   // [nb][tok_pad] activation scales, then [nb][tok_pad] scale * sum(q)
    int rows, rows_pad, nb, n_tok, tok_pad, mtiles;
    size_t qrow, cols;
};

// Issue this wave's share of the direct loads for chunk `chunk`. Rows,
// tokens and blocks past the end are clamped to the last valid one: they
// feed outputs that are never stored.
template <int DT, int KB>
__device__ __forceinline__ void issue_stage(GStage<DT, KB>& st, const GArgs& g, int chunk, int wave, int lane,
                                            int n0, int m0) {
    using P = GPlan<DT, KB>;
    constexpr int QB = GStage<DT, KB>::QB;
    const int b0 = chunk * KB;
#pragma unroll
    for (int k = 0; k < P::PER_WAVE; ++k) {
        const int ins = 4 * k + wave;  // instruction index within the stage, uniform per wave
        const void* src;
        lds_ptr_t dst;
        if (4 * k < P::I_A) {
            const int p = ins * 64 + lane;
            constexpr int per_blk = TILE * QB / 16;
            const int blk = p / per_blk, rem = p - blk * per_blk;
            const int row = QB == 32 ? rem >> 1 : rem, half = QB == 32 ? rem & 1 : 0;
            const int n = n0 + row < g.rows ? n0 + row : g.rows - 1;
            const int b = b0 + blk < g.nb ? b0 + blk : g.nb - 1;
            src = g.qs + (size_t)n * g.qrow + (size_t)b * QB + 16 * half;
            dst = (lds_ptr_t)&st.A[ins * 64 * 16];
        } else if (4 * k < P::I_A + P::I_B) {
            const int i = ins - P::I_A;
            const int p = i * 64 + lane;
            const int blk = p / (TILE * 2), rem = p - blk * TILE * 2;
            const int tok = rem >> 1, half = rem & 1;
            const int m = m0 + tok < g.n_tok ? m0 + tok : g.n_tok - 1;
            const int b = b0 + blk < g.nb ? b0 + blk : g.nb - 1;
            src = g.aq + (size_t)m * g.cols + (size_t)b * 32 + 16 * half;
            dst = (lds_ptr_t)&st.B[i * 64 * 16];
        } else {
            // Scale tables, [blk][TILE] f32 each: TILE / 4 pieces of 4 floats per block.
            const int i = ins - P::I_A - P::I_B;
            const int table = i / P::I_S, j = i - table * P::I_S;
            const int p = j * 64 + lane;
            const int blk = p / (TILE / 4), r4 = (p - blk * (TILE / 4)) * 4;
            const int b = b0 + blk < g.nb ? b0 + blk : g.nb - 1;
            float* base;
            if (table == 0) {
                src = g.swT + (size_t)b * g.rows_pad + n0 + r4;
                base = st.SW;
            } else if (table == 1) {
                src = g.sxT + (size_t)b * g.tok_pad + m0 + r4;
                base = st.SX;
            } else if (table == 2) {
                src = g.swT + (size_t)g.nb * g.rows_pad + (size_t)b * g.rows_pad + n0 + r4;
                base = st.BI;
            } else {
                src = g.sxT + (size_t)g.nb * g.tok_pad + (size_t)b * g.tok_pad + m0 + r4;
                base = st.SXQ;
            }
            dst = (lds_ptr_t)&base[j * 64 * 4];
        }
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
}

// s_waitcnt immediate with vmcnt = n (bits 3:0 and 15:14); expcnt and
// lgkmcnt at their maxima, so they do not wait.
#define NNH_VMCNT(n) ((((n)&0xF) | (0x7 << 4) | (0xF << 8) | ((((n) >> 4) & 0x3) << 14)))

template <int DT, int KB>
__device__ __forceinline__ void compute_stage(const GStage<DT, KB>& st, double (&acc)[2][2][16], int nblk, int wn,
                                              int wm, int h, int c) {
    constexpr int QB = GStage<DT, KB>::QB;
#pragma unroll
    for (int j = 0; j < KB; ++j) {
        if (j >= nblk) break;
        v4i av[2];
        float sw[2][16];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int rowA = wn * 64 + i * 32;
            int4 a;
            if (DT == 1) {
                a = *(const int4*)&st.A[(j * TILE + rowA + c) * QB + 16 * h];
            } else {
                const int4 q = *(const int4*)&st.A[(j * TILE + rowA + c) * QB];
                const int sh = 4 * h, mk = 0x0f0f0f0f;
                a.x = (int)((unsigned)q.x >> sh) & mk;
                a.y = (int)((unsigned)q.y >> sh) & mk;
                a.z = (int)((unsigned)q.z >> sh) & mk;
                a.w = (int)((unsigned)q.w >> sh) & mk;
            }
            av[i] = v4i{a.x, a.y, a.z, a.w};
            const float* swp = &st.SW[j * TILE + rowA + 4 * h];
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const float4 v = *(const float4*)(swp + 8 * gq);
                sw[i][4 * gq] = v.x;
                sw[i][4 * gq + 1] = v.y;
                sw[i][4 * gq + 2] = v.z;
                sw[i][4 * gq + 3] = v.w;
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int colB = wm * 64 + t * 32;
            const int4 bq = *(const int4*)&st.B[(j * TILE + colB + c) * 32 + 16 * h];
            const v4i bv = {bq.x, bq.y, bq.z, bq.w};
            const float sx = st.SX[j * TILE + colB + c];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                v16i z = {};
                const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv, z, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r)  // sw * sx is exact: 8 x 8 significant bits
                    acc[i][t][r] = __builtin_fma((double)P[r], (double)(sw[i][r] * sx), acc[i][t][r]);
            }
            if (DT == 2) {
                const double sxq = (double)st.SXQ[j * TILE + colB + c];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float* bip = &st.BI[j * TILE + wn * 64 + i * 32 + 4 * h];
#pragma unroll
                    for (int gq = 0; gq < 4; ++gq) {
                        const float4 v = *(const float4*)(bip + 8 * gq);
                        acc[i][t][4 * gq] = __builtin_fma((double)v.x, sxq, acc[i][t][4 * gq]);
                        acc[i][t][4 * gq + 1] = __builtin_fma((double)v.y, sxq, acc[i][t][4 * gq + 1]);
                        acc[i][t][4 * gq + 2] = __builtin_fma((double)v.z, sxq, acc[i][t][4 * gq + 2]);
                        acc[i][t][4 * gq + 3] = __builtin_fma((double)v.w, sxq, acc[i][t][4 * gq + 3]);
                    }
                }
            }
        }
    }
}

// One step of the ring: chunk c is in stage `cur`; chunk c + 2 goes into
// `nxt`, the stage chunk c - 1 was computed from.
template <int DT, int KB>
__device__ __forceinline__ void pipeline_step(GStage<DT, KB>& cur, GStage<DT, KB>& nxt, const GArgs& g, int c,
                                              int nchunks, double (&acc)[2][2][16], int wave, int lane, int n0,
                                              int m0, int wn, int wm, int h) {
    constexpr int L = GPlan<DT, KB>::PER_WAVE;
    if (c >= nchunks) return;
    // This wave's loads of chunk c are done once at most chunk c + 1's are outstanding.
    if (c + 1 < nchunks)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(L));
    else
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));
    // Every wave's loads of chunk c have landed, and every wave is done with
    // chunk c - 1. A bare barrier: __syncthreads() would also wait for the
    // loads still in flight for chunks c + 1 and c + 2.
    __builtin_amdgcn_s_barrier();
    if (c + 2 < nchunks) issue_stage<DT, KB>(nxt, g, c + 2, wave, lane, n0, m0);
    const int nblk = g.nb - c * KB < KB ? g.nb - c * KB : KB;
    compute_stage<DT, KB>(cur, acc, nblk, wn, wm, h, lane & 31);
}

template <int DT, int KB>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GArgs g, float* __restrict__ y, size_t y_stride) {
    __shared__ __attribute__((aligned(16))) GStage<DT, KB> s0, s1, s2;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, c = lane & 31;
    const int wn = wave >> 1, wm = wave & 1;  // 64-row, 64-token quadrant of the tile
    // Workgroups go round-robin to the 8 XCDs (one L2 each); renumber them so
    // that each XCD takes a contiguous range of row tiles and reads those
    // weights once, for every token tile.
    const int total = gridDim.x, per = total / 8, rem = total % 8;
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const int id = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    const int n0 = (id / g.mtiles) * TILE, m0 = (id % g.mtiles) * TILE;
    const int nchunks = (g.nb + KB - 1) / KB;

    double acc[2][2][16];  // [A tile][B tile][register]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][t][r] = 0.0;

    issue_stage<DT, KB>(s0, g, 0, wave, lane, n0, m0);
    if (nchunks > 1) issue_stage<DT, KB>(s1, g, 1, wave, lane, n0, m0);
    for (int ch = 0; ch < nchunks; ch += 3) {
        pipeline_step<DT, KB>(s0, s2, g, ch, nchunks, acc, wave, lane, n0, m0, wn, wm, h);
        pipeline_step<DT, KB>(s1, s0, g, ch + 1, nchunks, acc, wave, lane, n0, m0, wn, wm, h);
        pipeline_step<DT, KB>(s2, s1, g, ch + 2, nchunks, acc, wave, lane, n0, m0, wn, wm, h);
    }

#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int m = m0 + wm * 64 + t * 32 + c;
        if (m >= g.n_tok) continue;
        float* yr = y + (size_t)m * y_stride;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = n0 + wn * 64 + i * 32 + (r / 4) * 8 + 4 * h + (r % 4);
                if (n < g.rows) yr[n] = (float)acc[i][t][r];
            }
    }
}

// swT[b][n] = f32(scale[n][b]) and, for Q4, the biases in a second table
// after it; rows padded to a multiple of TILE with zeros.
__global__ void gemm_scales_kernel(const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
                                   float* __restrict__ swT, int rows, int rows_pad, int nb) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per = (size_t)rows_pad * nb;
    const int tables = bi ? 2 : 1;
    if (idx >= per * tables) return;
    const int tbl = (int)(idx / per);
    const size_t r = idx - tbl * per;
    const int b = (int)(r / rows_pad), n = (int)(r - (size_t)b * rows_pad);
    const uint16_t* src = tbl == 0 ? sc : bi;
    swT[idx] = n < rows ? bf16f(src[(size_t)n * nb + b]) : 0.0f;
}

}  // namespace

int gemm_rows_pad(int rows) { return (rows + TILE - 1) / TILE * TILE; }
int gemm_tok_pad(int n_tok) { return (n_tok + TILE - 1) / TILE * TILE; }

void launch_gemm_scales(const uint16_t* sc, const uint16_t* bi, float* swT, int rows, int nb, hipStream_t st) {
    const int rp = gemm_rows_pad(rows);
    const size_t n = (size_t)rp * nb * (bi ? 2 : 1);
    gemm_scales_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(sc, bi, swT, rows, rp, nb);
}

// Blocks per ring stage.
constexpr int GEMM_KB = 4;

void launch_gemm_i8(int dtype, const uint8_t* qs, const float* swT, const int8_t* aq, const float* sxT, int rows,
                    int nb, int n_tok, float* y, size_t y_stride, hipStream_t st) {
    GArgs g;
    g.qs = qs;
    g.swT = swT;
    g.aq = aq;
    g.sxT = sxT;
    g.rows = rows;
    g.rows_pad = gemm_rows_pad(rows);
    g.nb = nb;
    g.n_tok = n_tok;
    g.tok_pad = gemm_tok_pad(n_tok);
    g.mtiles = ceil_div(n_tok, TILE);
    g.cols = (size_t)nb * 32;
    g.qrow = dtype == 1 ? g.cols : g.cols / 2;
    const dim3 grid(g.mtiles * ceil_div(rows, TILE)), block(256);
    if (dtype == 1)
        gemm_i8_kernel<1, GEMM_KB><<<grid, block, 0, st>>>(g, y, y_stride);
    else
        gemm_i8_kernel<2, GEMM_KB><<<grid, block, 0, st>>>(g, y, y_stride);
}

}  // namespace nnh
