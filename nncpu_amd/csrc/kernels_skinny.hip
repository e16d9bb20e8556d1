// The int8 matmul for a few activation vectors (5..16: batched speculative
// verify, short prompts) on the matrix unit: a weight stream with a
// 32-token MFMA.
//
// One v_mfma_i32_32x32x32_i8 per (32 weight rows, block): A = the
// activations (MFMA rows i = tokens, padded to 32 by repeating the last
// one), B = the weights (MFMA columns j = weight rows). Result element
// (i, j) sits in lane j + 32h, register r with i = (r/4)*8 + 4h + r%4, so
// tokens 0..7 are registers 0..3 and tokens 8..15 registers 4..7 of every
// lane: only NR = 4 or 8 registers per lane carry real outputs, and the
// scaling epilogue runs on those alone. The block dot products are exact;
// the epilogue is the GEMM's (exact scale products from a two-block f32
// outer-product MFMA, f64 accumulation), so every output is within one f32
// ulp of the exact sum.
//
// Workgroup: 4 waves on 32 weight rows; the waves split the blocks into
// contiguous ranges and stream them straight into registers (16 bytes per
// lane and block, nontemporal), four blocks per group, double-buffered. Partial sums
// meet in LDS and are added in wave order. Matrices with few row groups are
// split along K over several workgroups as well; those partials go to a
// workspace (f64) and a second kernel adds them in split order.

#include "common.h"

namespace nnh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int SK_W = 4;           // waves per workgroup
constexpr int SK_G = 4;           // blocks per load group (even: scale products go in pairs)
constexpr int SK_MAX_SPLITS = 8;  // K-split workgroups per row group

struct KArgs {
    const uint8_t* qs;  // weights, nncpu row-major quants
    const float* swT;   // [nb][rows_pad] weight scales; Q4 biases follow at + nb * rows_pad
    const int8_t* aq;   // activation quants [n_tok][cols]
    const float* sxT;   // [nb][tok_pad] activation scales, then [nb][tok_pad] scale * sum(q)
    double* ws;         // K-split partials [split][16][rows_pad] (ksplit > 1)
    int rows, rows_pad, nb, n_tok, tok_pad, ksplit;
    size_t qrow, cols;
};

// One load group: the lane's 16 weight and 16 activation bytes of SK_G
// blocks, and the scales of the pair members it contributes to the outer
// products (lane half h gives block 2p + h of pair p).
template <int DT>
struct Group {
    int4 w[SK_G], a[SK_G];
    float sw[SK_G / 2], sx[SK_G / 2];
    float bi[DT == 2 ? SK_G : 1], sxq[DT == 2 ? SK_G / 2 : 1];
};

template <int DT>
__device__ __forceinline__ void load_group(Group<DT>& gr, const KArgs& g, const uint8_t* wrow, const int8_t* arow,
                                           int b0, int kb1, int n0, int h, int c) {
#pragma unroll
    for (int k = 0; k < SK_G; ++k) {
        const int b = b0 + k < kb1 ? b0 + k : kb1 - 1;  // past the range: reload the last block, unused
        if (DT == 1)
            gr.w[k] = load_nt16(wrow + (size_t)b * 32 + 16 * h);
        else
            gr.w[k] = load_nt16(wrow + (size_t)b * 16);
        gr.a[k] = *(const int4*)(arow + (size_t)b * 32 + 16 * h);
        if (DT == 2) gr.bi[k] = g.swT[(size_t)g.nb * g.rows_pad + (size_t)b * g.rows_pad + n0 + c];
    }
#pragma unroll
    for (int p = 0; p < SK_G / 2; ++p) {
        const int b = b0 + 2 * p + h < kb1 ? b0 + 2 * p + h : kb1 - 1;
        gr.sw[p] = g.swT[(size_t)b * g.rows_pad + n0 + c];
        gr.sx[p] = g.sxT[(size_t)b * g.tok_pad + c];
        if (DT == 2) gr.sxq[p] = g.sxT[(size_t)g.nb * g.tok_pad + (size_t)b * g.tok_pad + c];
    }
}

template <int DT, int NR>
__device__ __forceinline__ void compute_group(const Group<DT>& gr, double (&acc)[NR], int nblk, int h) {
#pragma unroll
    for (int p = 0; p < SK_G / 2; ++p) {
        if (2 * p >= nblk) break;
        const v32f z = {};
        // s_x[token i] * s_w[row j] for blocks 2p and 2p + 1, exact in f32.
        const v32f S = __builtin_amdgcn_mfma_f32_32x32x1f32(gr.sx[p], gr.sw[p], z, 0, 0, 0);
        v32f Q;
        if (DT == 2) Q = __builtin_amdgcn_mfma_f32_32x32x1f32(gr.sxq[p], 1.0f, z, 0, 0, 0);  // s_x sum(q_x) [i]
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int k = 2 * p + jj;
            if (k >= nblk) break;
            int4 w = gr.w[k];
            if (DT == 2) {
                const int sh = 4 * h, mk = 0x0f0f0f0f;
                w.x = (int)((unsigned)w.x >> sh) & mk;
                w.y = (int)((unsigned)w.y >> sh) & mk;
                w.z = (int)((unsigned)w.z >> sh) & mk;
                w.w = (int)((unsigned)w.w >> sh) & mk;
            }
            const v16i zi = {};
            const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(v4i{gr.a[k].x, gr.a[k].y, gr.a[k].z, gr.a[k].w},
                                                                 v4i{w.x, w.y, w.z, w.w}, zi, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r] = __builtin_fma((double)P[r], (double)S[16 * jj + r], acc[r]);
            if (DT == 2) {
                const double bi = (double)gr.bi[k];  // bias[row] * (s_x sum q_x)[token], exact in f64
#pragma unroll
                for (int r = 0; r < NR; ++r) acc[r] = __builtin_fma(bi, (double)Q[16 * jj + r], acc[r]);
            }
        }
    }
}

template <int DT, int NR>
__global__ __launch_bounds__(SK_W * 64) void skinny_i8_kernel(KArgs g, float* __restrict__ y, size_t y_stride) {
    __shared__ double red[SK_W][NR][64];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, c = lane & 31;
    const int rg = blockIdx.x / g.ksplit, ks = blockIdx.x % g.ksplit;
    const int n0 = rg * 32;
    const int n = n0 + c < g.rows ? n0 + c : g.rows - 1;  // rows and tokens past the end repeat the last
    const int m = c < g.n_tok ? c : g.n_tok - 1;
    const int parts = g.ksplit * SK_W, part = ks * SK_W + wave;
    const int kb0 = (int)((long)part * g.nb / parts), kb1 = (int)((long)(part + 1) * g.nb / parts);
    const uint8_t* wrow = g.qs + (size_t)n * g.qrow;
    const int8_t* arow = g.aq + (size_t)m * g.cols;

    double acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0;
    if (kb1 > kb0) {
        const int ngroups = (kb1 - kb0 + SK_G - 1) / SK_G;
        Group<DT> ga, gb;
        load_group<DT>(ga, g, wrow, arow, kb0, kb1, n0, h, c);
        for (int gi = 0; gi < ngroups; gi += 2) {
            const int b0 = kb0 + gi * SK_G;
            if (gi + 1 < ngroups) load_group<DT>(gb, g, wrow, arow, b0 + SK_G, kb1, n0, h, c);
            compute_group<DT, NR>(ga, acc, kb1 - b0, h);
            if (gi + 1 >= ngroups) break;
            if (gi + 2 < ngroups) load_group<DT>(ga, g, wrow, arow, b0 + 2 * SK_G, kb1, n0, h, c);
            compute_group<DT, NR>(gb, acc, kb1 - b0 - SK_G, h);
        }
    }

#pragma unroll
    for (int r = 0; r < NR; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    // Thread (r, l) finishes result register r of lane l: the SK_W * 64
    // threads cover the NR * 64 outputs in NR / SK_W rounds.
    static_assert(NR % SK_W == 0, "whole rounds");
    const int l = tid & 63;
    const int row = n0 + (l & 31);
#pragma unroll
    for (int r = tid >> 6; r < NR; r += SK_W) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < SK_W; ++w) s += red[w][r][l];
        const int i = (r / 4) * 8 + 4 * (l >> 5) + (r % 4);  // token
        if (i < g.n_tok && row < g.rows) {
            if (g.ksplit == 1)
                y[(size_t)i * y_stride + row] = (float)s;
            else
                g.ws[((size_t)ks * 16 + i) * g.rows_pad + row] = s;
        }
    }
}

// y = the sum of the K-split partials in split order (f64), rounded once.
// All partials are loaded before the first add, so their latencies overlap.
__global__ void skinny_reduce_kernel(const double* __restrict__ ws, int ksplit, int rows, int rows_pad, int n_tok,
                                     float* __restrict__ y, size_t y_stride) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
    if (row >= rows) return;
    double p[SK_MAX_SPLITS];
#pragma unroll
    for (int k = 0; k < SK_MAX_SPLITS; ++k) p[k] = k < ksplit ? ws[((size_t)k * 16 + i) * rows_pad + row] : 0.0;
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < SK_MAX_SPLITS; ++k)
        if (k < ksplit) s += p[k];
    y[(size_t)i * y_stride + row] = (float)s;
}

}  // namespace

// K-split over workgroups when the row groups alone do not cover the CUs;
// each wave keeps at least two blocks.
int skinny_splits(int rows, int nb) {
    const int groups = ceil_div(rows, 32);
    if (groups >= 160) return 1;
    int ks = ceil_div(256, groups);
    const int most = nb / (2 * SK_W);
    if (ks > most) ks = most;
    if (ks > SK_MAX_SPLITS) ks = SK_MAX_SPLITS;
    return ks < 1 ? 1 : ks;
}

size_t skinny_workspace_bytes(int rows, int nb) {
    const int ks = skinny_splits(rows, nb);
    return ks == 1 ? 0 : (size_t)ks * 16 * gemm_rows_pad(rows) * sizeof(double);
}

void launch_skinny_i8(int dtype, const uint8_t* qs, const float* swT, const int8_t* aq, const float* sxT, int rows,
                      int nb, int n_tok, float* y, size_t y_stride, double* ws, hipStream_t st) {
    KArgs g;
    g.qs = qs;
    g.swT = swT;
    g.aq = aq;
    g.sxT = sxT;
    g.ws = ws;
    g.rows = rows;
    g.rows_pad = gemm_rows_pad(rows);
    g.nb = nb;
    g.n_tok = n_tok;
    g.tok_pad = gemm_tok_pad(n_tok);
    g.ksplit = skinny_splits(rows, nb);
    g.cols = (size_t)nb * 32;
    g.qrow = dtype == 1 ? g.cols : g.cols / 2;
    const dim3 grid(ceil_div(rows, 32) * g.ksplit), block(SK_W * 64);
#define NNH_SK(DT, NR) skinny_i8_kernel<DT, NR><<<grid, block, 0, st>>>(g, y, y_stride)
    if (dtype == 1) {
        if (n_tok <= 8) NNH_SK(1, 4); else NNH_SK(1, 8);
    } else {
        if (n_tok <= 8) NNH_SK(2, 4); else NNH_SK(2, 8);
    }
#undef NNH_SK
    if (g.ksplit > 1)
        skinny_reduce_kernel<<<dim3(ceil_div(rows, 256), n_tok), 256, 0, st>>>(ws, g.ksplit, rows, g.rows_pad, n_tok, y,
                                                                               y_stride);
}

}  // namespace nnh
